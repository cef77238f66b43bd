// Instance normalisation + LeakyReLU for channels-last (B, S, C) float32 tensors.
//
// Three bandwidth-bound launches (two full reads and one write of the tensor):
//   1. norm_stats: each workgroup owns one chunk of R*vpi voxels of one sample and keeps
//      its values in registers; it reduces the chunk sum (wavefront shuffles + LDS),
//      forms the chunk mean, then the centred sum of squares from the same registers
//      (two-pass inside the chunk) and writes (mean, M2) per channel.
//   2. norm_merge: per (b, c), the chunk partials are combined with Chan's parallel
//      update in float64, giving mean and biased variance of x + input_bias.
//   3. norm_apply: y = max(slope*r, r), r = fma(x + b - mean, gamma*rsqrt(var+eps), beta)
//      (+ residual before the activation), vectorised float4, in place allowed.
#include <mutex>

#include "nnx_internal.h"

namespace nnx {
namespace {

constexpr int kRows = 16;       // voxels per thread in the statistics pass
constexpr int kMaxThreads = 256;

template <int VW>
struct Vec;
template <>
struct Vec<4> {
  typedef float type __attribute__((ext_vector_type(4)));
};
template <>
struct Vec<1> {
  typedef float type;
};

template <int VW>
__device__ __forceinline__ float lane_of(const typename Vec<VW>::type& v, int q) {
  if constexpr (VW == 1) {
    return v;
  } else {
    return v[q];
  }
}

template <int VW>
__global__ __launch_bounds__(kMaxThreads) void norm_stats_kernel(
    const float* __restrict__ x, const float* __restrict__ in_bias, float2* __restrict__ partial,
    int64_t S, int C, int vpi, int nchunks) {
  typedef typename Vec<VW>::type V;
  __shared__ float red[kMaxThreads * VW];
  __shared__ float cmean[kMaxThreads * VW];
  const int b = blockIdx.y;
  const int chunk = blockIdx.x;
  const int groups = C / VW;
  const int tid = threadIdx.x;
  const bool active = tid < vpi * groups;
  const int g = tid % groups;
  const int j = tid / groups;
  const int64_t v0 = (int64_t)chunk * kRows * vpi;
  const int64_t nvalid64 = S - v0 < (int64_t)kRows * vpi ? S - v0 : (int64_t)kRows * vpi;
  const float n = (float)nvalid64;
  const float* xs = x + (int64_t)b * S * C;

  float bias[VW];
#pragma unroll
  for (int q = 0; q < VW; ++q) bias[q] = (in_bias && active) ? in_bias[g * VW + q] : 0.f;

  float vals[kRows][VW];
  bool valid[kRows];
  float sum[VW];
#pragma unroll
  for (int q = 0; q < VW; ++q) sum[q] = 0.f;
#pragma unroll
  for (int it = 0; it < kRows; ++it) {
    const int64_t v = v0 + (int64_t)it * vpi + j;
    valid[it] = active && v < S;
    V raw;
    if (valid[it]) {
      raw = *reinterpret_cast<const V*>(xs + v * C + g * VW);
    } else {
      if constexpr (VW == 1) raw = 0.f; else raw = V{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int q = 0; q < VW; ++q) {
      float val = lane_of<VW>(raw, q);
      if (in_bias) val = val + bias[q];
      vals[it][q] = valid[it] ? val : 0.f;
      sum[q] += vals[it][q];
    }
  }
#pragma unroll
  for (int q = 0; q < VW; ++q) red[tid * VW + q] = sum[q];
  __syncthreads();
  if (tid < groups) {
#pragma unroll
    for (int q = 0; q < VW; ++q) {
      float t = 0.f;
      for (int jj = 0; jj < vpi; ++jj) t += red[(jj * groups + tid) * VW + q];
      cmean[tid * VW + q] = t / n;
    }
  }
  __syncthreads();
  float m2[VW];
#pragma unroll
  for (int q = 0; q < VW; ++q) {
    const float mu = active ? cmean[g * VW + q] : 0.f;
    float acc = 0.f;
#pragma unroll
    for (int it = 0; it < kRows; ++it) {
      const float d = valid[it] ? vals[it][q] - mu : 0.f;
      acc = fmaf(d, d, acc);
    }
    m2[q] = acc;
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < VW; ++q) red[tid * VW + q] = m2[q];
  __syncthreads();
  if (tid < groups) {
#pragma unroll
    for (int q = 0; q < VW; ++q) {
      float t = 0.f;
      for (int jj = 0; jj < vpi; ++jj) t += red[(jj * groups + tid) * VW + q];
      partial[((int64_t)b * nchunks + chunk) * C + tid * VW + q] =
          make_float2(cmean[tid * VW + q], t);
    }
  }
}

// Chan et al. pairwise combination of (count, mean, M2) in float64.
__device__ __forceinline__ void chan_merge(double& na, double& ma, double& m2a, double nb,
                                           double mb, double m2b) {
  if (nb == 0.0) return;
  if (na == 0.0) {
    na = nb;
    ma = mb;
    m2a = m2b;
    return;
  }
  const double n = na + nb;
  const double delta = mb - ma;
  ma = ma + delta * (nb / n);
  m2a = m2a + m2b + delta * delta * (na * nb / n);
  na = n;
}

__global__ __launch_bounds__(256) void norm_merge_kernel(const float2* __restrict__ partial,
                                                         float4* __restrict__ params,
                                                         const float* __restrict__ beta,
                                                         const float* __restrict__ gamma,
                                                         int64_t S, int C, int nchunks,
                                                         int chunk_vox, float eps) {
  __shared__ double sn[256], sm[256], s2[256];
  const int c = blockIdx.x;
  const int b = blockIdx.y;
  double n = 0.0, m = 0.0, m2 = 0.0;
  for (int i = threadIdx.x; i < nchunks; i += blockDim.x) {
    const int64_t start = (int64_t)i * chunk_vox;
    const double cnt = (double)((S - start) < chunk_vox ? (S - start) : chunk_vox);
    const float2 p = partial[((int64_t)b * nchunks + i) * C + c];
    chan_merge(n, m, m2, cnt, (double)p.x, (double)p.y);
  }
  sn[threadIdx.x] = n;
  sm[threadIdx.x] = m;
  s2[threadIdx.x] = m2;
  __syncthreads();
  for (int stride = blockDim.x / 2; stride > 0; stride >>= 1) {
    if ((int)threadIdx.x < stride) {
      double na = sn[threadIdx.x], ma = sm[threadIdx.x], m2a = s2[threadIdx.x];
      chan_merge(na, ma, m2a, sn[threadIdx.x + stride], sm[threadIdx.x + stride],
                 s2[threadIdx.x + stride]);
      sn[threadIdx.x] = na;
      sm[threadIdx.x] = ma;
      s2[threadIdx.x] = m2a;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const double var = s2[0] / (double)S;
    float varf = (float)(var > 0.0 ? var : 0.0);
    float scale = 1.0f / sqrtf(varf + eps);
    if (gamma) scale = gamma[c] * scale;
    params[(int64_t)b * C + c] = make_float4((float)sm[0], scale, beta ? beta[c] : 0.f, 0.f);
  }
}

// Same merge for partials that carry their own counts (per-tile partials written by the
// convolution epilogue: (mean, M2, n, 0) at partial[(b * nparts + i) * C + c]), in two passes.
// Pass 1: block (j, b) of S = gridDim.x blocks merges rows [slice_row(j), slice_row(j + 1))
// of item b, slice_row(j) = floor(j * nparts / S): balanced slices (their lengths differ by
// at most one row), each at least two rows long when nparts >= 2 S, so every slice has two
// rows to hold its result; a thread takes
// channel cb + t % CB of every G-th row (CB = min(C, 256) channels a pass, G = 256 / CB
// row groups), so each row is read as one contiguous run; the groups are merged through
// LDS, and the slice's (mean, M2) in float64 and its count are written over the slice's
// own first two rows (read by this block only, and no longer needed).
__device__ __forceinline__ int64_t slice_row(int j, int nparts, int nslices) {
  return (int64_t)j * nparts / nslices;
}

__global__ __launch_bounds__(256) void norm_merge_slices_kernel(float4* __restrict__ partial, int C,
                                                                int nparts) {
  __shared__ double sn[256], sm[256], s2[256];
  const int j = blockIdx.x, b = blockIdx.y;
  const int t = threadIdx.x;
  const int CB = C < 256 ? C : 256;
  const int G = 256 / CB;
  const int g = t / CB;
  const int r0 = (int)slice_row(j, nparts, gridDim.x);
  const int r1 = (int)slice_row(j + 1, nparts, gridDim.x);
  float4* rows = partial + (int64_t)b * nparts * C;
  // (mean, M2) as a double pair and the count, per channel of this pass
  double res_m[2], res_2[2];
  float res_n[2];
  int npass = 0;
  for (int cb = 0; cb < C; cb += CB, ++npass) {
    const int c = cb + t % CB;
    const bool active = g < G && c < C;
    double n = 0.0, m = 0.0, m2 = 0.0;
    if (active) {
      int r = r0 + g;
      // four rows in flight per step
      for (; r + 3 * G < r1; r += 4 * G) {
        float4 p[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) p[q] = rows[(int64_t)(r + q * G) * C + c];
#pragma unroll
        for (int q = 0; q < 4; ++q) chan_merge(n, m, m2, (double)p[q].z, (double)p[q].x, (double)p[q].y);
      }
      for (; r < r1; r += G) {
        const float4 p = rows[(int64_t)r * C + c];
        chan_merge(n, m, m2, (double)p.z, (double)p.x, (double)p.y);
      }
    }
    sn[t] = n;
    sm[t] = m;
    s2[t] = m2;
    __syncthreads();
    // groups g = 1 .. G-1 into group 0, one thread per channel
    if (t < CB) {
      double na = sn[t], ma = sm[t], m2a = s2[t];
      for (int q = 1; q < G; ++q) chan_merge(na, ma, m2a, sn[q * CB + t], sm[q * CB + t], s2[q * CB + t]);
      if (npass < 2) {
        res_m[npass] = ma;
        res_2[npass] = m2a;
        res_n[npass] = (float)na;
      }
    }
    __syncthreads();
  }
  // every read of the slice is done: row r0 holds (mean, M2) as doubles, row r0 + 1 the count
  if (t < CB) {
    for (int q = 0; q < npass && q < 2; ++q) {
      const int c = q * CB + t;
      if (c < C) {
        double2* out = reinterpret_cast<double2*>(rows + (int64_t)r0 * C + c);
        *out = make_double2(res_m[q], res_2[q]);
        rows[(int64_t)(r0 + 1) * C + c] = make_float4(res_n[q], 0.f, 0.f, 0.f);
      }
    }
  }
}

// Pass 2: a wave per (b, c) (four a workgroup): lane l merges entries l, l + 64, ... in
// order, then the lanes' results merge along a fixed butterfly (lower lane first at every
// level), and lane 0 writes the parameters.  With `raw` (at most 64 partial rows: no pass 1)
// the entries are the partial rows themselves, else the slices' results.
__device__ __forceinline__ double shfl_xor_f64(double v, int o) {
  const int lo = __shfl_xor((int)(__double_as_longlong(v) & 0xffffffffLL), o);
  const int hi = __shfl_xor((int)(__double_as_longlong(v) >> 32), o);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

__global__ __launch_bounds__(256) void norm_merge_final_kernel(const float4* __restrict__ partial,
                                                               float4* __restrict__ params,
                                                               const float* __restrict__ beta,
                                                               const float* __restrict__ gamma,
                                                               int64_t S, int C, int nparts,
                                                               int nslices, int raw,
                                                               float eps) {
  const int lane = threadIdx.x & 63;
  const int c = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int b = blockIdx.y;
  if (c >= C) return;  // uniform over the wave; the kernel has no barrier
  const float4* rows = partial + (int64_t)b * nparts * C;
  double n = 0.0, m = 0.0, m2 = 0.0;
  const int count = raw ? nparts : nslices;
  for (int j = lane; j < count; j += 64) {
    double en, em, e2;
    if (raw) {
      const float4 p = rows[(int64_t)j * C + c];
      en = p.z;
      em = p.x;
      e2 = p.y;
    } else {
      const int64_t r0 = slice_row(j, nparts, nslices);
      const double2 mv = *reinterpret_cast<const double2*>(rows + r0 * C + c);
      en = rows[(r0 + 1) * C + c].x;
      em = mv.x;
      e2 = mv.y;
    }
    chan_merge(n, m, m2, en, em, e2);
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const double on = shfl_xor_f64(n, o), om = shfl_xor_f64(m, o), o2 = shfl_xor_f64(m2, o);
    if (lane & o) {
      // the partner is the lower lane: its entries come first
      double pn = on, pm = om, p2 = o2;
      chan_merge(pn, pm, p2, n, m, m2);
      n = pn;
      m = pm;
      m2 = p2;
    } else {
      chan_merge(n, m, m2, on, om, o2);
    }
  }
  if (lane != 0) return;
  const double var = m2 / (double)S;
  float varf = (float)(var > 0.0 ? var : 0.0);
  float scale = 1.0f / sqrtf(varf + eps);
  if (gamma) scale = gamma[c] * scale;
  params[(int64_t)b * C + c] = make_float4((float)m, scale, beta ? beta[c] : 0.f, 0.f);
}

// y = act(fma(x (+ bias) - mean, scale, beta) (+ residual)) over a (B, S, C) tensor, VW
// channels a vector.  A workgroup streams runs of kRun = 4 * 256 consecutive vectors of one
// item (thread t takes vectors t, t + 256, t + 512, t + 768 of the run, all four loads
// issued before the arithmetic), runs gridDim.x apart; the channel of each vector follows
// from the run's first channel (advanced by the run stride modulo C) and the thread's four
// fixed offsets, and the parameters come from LDS.  y may alias x.
template <int VW>
__global__ __launch_bounds__(256) void norm_apply_kernel(
    const float* x, float* y, const float4* __restrict__ params, const float* __restrict__ in_bias,
    const float* residual, int64_t SC, int C, int act, float slope) {
  typedef typename Vec<VW>::type V;
  constexpr int kUnroll = 4, kRun = kUnroll * 256;
  extern __shared__ float smem[];  // C * 4: mean, scale, beta, input bias
  float* s_mean = smem;
  float* s_scale = smem + C;
  float* s_beta = smem + 2 * C;
  float* s_bias = smem + 3 * C;
  const int b = blockIdx.y;
  for (int i = threadIdx.x; i < C; i += blockDim.x) {
    const float4 p = params[(int64_t)b * C + i];
    s_mean[i] = p.x;
    s_scale[i] = p.y;
    s_beta[i] = p.z;
    s_bias[i] = in_bias ? in_bias[i] : 0.f;
  }
  __syncthreads();
  const float* xs = x + (int64_t)b * SC;
  float* ys = y + (int64_t)b * SC;
  const float* rs = residual ? residual + (int64_t)b * SC : nullptr;
  const int64_t nvec = SC / VW;
  const bool has_bias = in_bias != nullptr;
  const int tid = threadIdx.x;
  // channel offsets of the thread's four vectors within a run, and the run's first channel
  int cu[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) cu[u] = (int)(((int64_t)(u * 256 + tid) * VW) % C);
  int64_t run = blockIdx.x;
  int crun = (int)((run * kRun * VW) % C);
  const int dcrun = (int)(((int64_t)gridDim.x * kRun * VW) % C);
  auto apply = [&](V xv, V rv, int cb) {
    V out;
#pragma unroll
    for (int q = 0; q < VW; ++q) {
      const int c = cb + q;
      float v = lane_of<VW>(xv, q);
      if (has_bias) v = v + s_bias[c];
      float r = fmaf(v - s_mean[c], s_scale[c], s_beta[c]);
      if (rs) r = r + lane_of<VW>(rv, q);
      if (act) r = fmaxf(slope * r, r);
      if constexpr (VW == 1) out = r; else out[q] = r;
    }
    return out;
  };
  auto chan = [&](int u) {
    const int c = crun + cu[u];
    return c >= C ? c - C : c;
  };
  for (; (run + 1) * kRun <= nvec; run += gridDim.x) {
    const int64_t v0 = run * kRun + tid;
    V xv[kUnroll], rv[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      xv[u] = *reinterpret_cast<const V*>(xs + (v0 + u * 256) * VW);
      if (rs) rv[u] = *reinterpret_cast<const V*>(rs + (v0 + u * 256) * VW);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      *reinterpret_cast<V*>(ys + (v0 + u * 256) * VW) = apply(xv[u], rs ? rv[u] : xv[u], chan(u));
    crun += dcrun;
    if (crun >= C) crun -= C;
  }
  // the partial last run
  if (run * kRun < nvec) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t v = run * kRun + u * 256 + tid;
      if (v < nvec) {
        const V xv = *reinterpret_cast<const V*>(xs + v * VW);
        const V rv = rs ? *reinterpret_cast<const V*>(rs + v * VW) : xv;
        *reinterpret_cast<V*>(ys + v * VW) = apply(xv, rv, chan(u));
      }
    }
  }
}

// Average pooling with kernel = stride (kd, kh, kw) of an NDHWC tensor.  Block (x, y, z) =
// (run of 256 (output x, channel group) pairs, output y, item * od + output z); a thread
// sums its window of VW-channel vectors in (a, e, f) order, then multiplies by 1 / (kd kh kw).
template <int VW>
__global__ __launch_bounds__(256) void avgpool_kernel(const float* __restrict__ x,
                                                      float* __restrict__ y, int D, int H, int W,
                                                      int C, int kd, int kh, int kw) {
  typedef typename Vec<VW>::type V;
  const int od = D / kd, oh = H / kh, ow = W / kw;
  const int cg = C / VW;
  const int ix = blockIdx.x * 256 + threadIdx.x;
  if (ix >= ow * cg) return;
  const int xx = ix / cg, c = (ix - xx * cg) * VW;
  const int yy = blockIdx.y;
  const int zz = blockIdx.z % od;
  const int64_t b = blockIdx.z / od;
  const float inv = 1.0f / (float)(kd * kh * kw);
  V s;
  if constexpr (VW == 1) s = 0.f; else s = V{0.f, 0.f, 0.f, 0.f};
  for (int a = 0; a < kd; ++a)
    for (int e = 0; e < kh; ++e)
      for (int f = 0; f < kw; ++f)
        s += *reinterpret_cast<const V*>(
            x + ((((b * D) + zz * kd + a) * H + yy * kh + e) * (int64_t)W + xx * kw + f) * C + c);
  *reinterpret_cast<V*>(y + (((b * od + zz) * oh + yy) * (int64_t)ow + xx) * C + c) = s * inv;
}

// Centred crop / zero pad of an NDHWC tensor: out[b, z, y, x, c] = in[b, z + oz, y + oy,
// x + ox, c] inside the input, 0 outside; offsets o = (in - out) / 2 truncated toward
// zero (crop start delta // 2, or pad before (-delta) // 2).  VW channels per thread.
template <int VW>
__global__ __launch_bounds__(256) void match_spatial_kernel(const float* __restrict__ x,
                                                            float* __restrict__ y, int64_t nout,
                                                            int ID, int IH, int IW, int OD,
                                                            int OH, int OW, int C, int oz,
                                                            int oy, int ox) {
  typedef float V __attribute__((ext_vector_type(VW)));
  const int cv = C / VW;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nout;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % cv) * VW;
    int64_t v = i / cv;
    const int xx = (int)(v % OW) + ox;
    v /= OW;
    const int yy = (int)(v % OH) + oy;
    v /= OH;
    const int zz = (int)(v % OD) + oz;
    const int64_t b = v / OD;
    V r = {};
    if ((unsigned)zz < (unsigned)ID && (unsigned)yy < (unsigned)IH && (unsigned)xx < (unsigned)IW)
      r = *reinterpret_cast<const V*>(x + (((b * ID + zz) * IH + yy) * (int64_t)IW + xx) * C + c);
    *reinterpret_cast<V*>(y + i * VW) = r;
  }
}

__global__ __launch_bounds__(256) void nonfinite_kernel(const float* __restrict__ x, int64_t n,
                                                        unsigned int* count) {
  __shared__ unsigned int total;
  if (threadIdx.x == 0) total = 0;
  __syncthreads();
  unsigned int local = 0;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    local += isfinite(x[i]) ? 0u : 1u;
  if (local) atomicAdd(&total, local);
  __syncthreads();
  if (threadIdx.x == 0 && total) atomicAdd(count, total);
}

__global__ void fill_zero_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

__global__ void fill_zero_bytes_kernel(unsigned char* p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

struct StatsLayout {
  int vw, groups, vpi, chunk_vox;
  int64_t nchunks;
};

StatsLayout stats_layout(int64_t spatial, int channels) {
  StatsLayout l;
  l.vw = channels % 4 == 0 ? 4 : 1;
  l.groups = channels / l.vw;
  require(l.groups <= kMaxThreads, "instance normalisation supports at most 1024 channels");
  l.vpi = kMaxThreads / l.groups;
  l.chunk_vox = kRows * l.vpi;
  l.nchunks = ceil_div(spatial, l.chunk_vox);
  return l;
}

}  // namespace

size_t instnorm_workspace_bytes(int batch, int64_t spatial, int channels) {
  // the limits instnorm_params enforces; they also keep the byte count below 2^61
  require(batch >= 1 && spatial >= 1 && channels >= 1, "instance normalisation needs a non-empty tensor");
  require(batch <= 65535, "instance normalisation batch too large");
  const StatsLayout l = stats_layout(spatial, channels);
  require(l.nchunks < (1LL << 31), "instance normalisation tensor too large");
  const size_t partial = (size_t)batch * l.nchunks * channels * sizeof(float2);
  const size_t params = (size_t)batch * channels * sizeof(float4);
  return ((partial + 255) / 256) * 256 + params;
}

void instnorm_params(const float* x, int batch, int64_t spatial, int channels,
                     const float* input_bias, const float* gamma, const float* beta, float eps,
                     void* ws, size_t ws_bytes, float4* params, hipStream_t st) {
  require(x != nullptr, "instance normalisation pointers must not be null");
  require(batch >= 1 && spatial >= 1 && channels >= 1, "instance normalisation needs a non-empty tensor");
  require(eps > 0.f, "instance-normalization epsilon must be positive");
  require(batch <= 65535, "instance normalisation batch too large");
  const StatsLayout l = stats_layout(spatial, channels);
  require(l.nchunks < (1LL << 31), "instance normalisation tensor too large");
  require(ws && ws_bytes >= instnorm_workspace_bytes(batch, spatial, channels),
          "instance normalisation workspace too small");
  float2* partial = reinterpret_cast<float2*>(ws);
  const size_t partial_bytes = (size_t)batch * l.nchunks * channels * sizeof(float2);
  if (!params)
    params = reinterpret_cast<float4*>(reinterpret_cast<char*>(ws) +
                                       ((partial_bytes + 255) / 256) * 256);
  const dim3 sgrid((unsigned)l.nchunks, (unsigned)batch);
  const double nelem = (double)batch * spatial * channels;
  {
  ProfScope prof("instnorm_stats", 0.0, 4.0 * nelem, st);
  if (l.vw == 4)
    hipLaunchKernelGGL(norm_stats_kernel<4>, sgrid, dim3(kMaxThreads), 0, st, x, input_bias,
                       partial, spatial, channels, l.vpi, (int)l.nchunks);
  else
    hipLaunchKernelGGL(norm_stats_kernel<1>, sgrid, dim3(kMaxThreads), 0, st, x, input_bias,
                       partial, spatial, channels, l.vpi, (int)l.nchunks);
  launch_check("instnorm stats");
  }
  {
  ProfScope prof("instnorm_merge", 0.0, 8.0 * (double)batch * l.nchunks * channels, st);
  hipLaunchKernelGGL(norm_merge_kernel, dim3(channels, batch), dim3(256), 0, st, partial, params,
                     beta, gamma, spatial, channels, (int)l.nchunks, l.chunk_vox, eps);
  launch_check("instnorm merge");
  }
}

void instnorm_lrelu(const float* x, float* y, int batch, int64_t spatial, int channels,
                    const float* input_bias, const float* gamma, const float* beta, float eps,
                    bool act, float slope, const float* residual, void* ws, size_t ws_bytes,
                    hipStream_t st) {
  require(x && y, "instance normalisation pointers must not be null");
  instnorm_params(x, batch, spatial, channels, input_bias, gamma, beta, eps, ws, ws_bytes,
                  nullptr, st);
  const StatsLayout l = stats_layout(spatial, channels);
  const size_t partial_bytes = (size_t)batch * l.nchunks * channels * sizeof(float2);
  const float4* params = reinterpret_cast<const float4*>(reinterpret_cast<char*>(ws) +
                                                         ((partial_bytes + 255) / 256) * 256);
  instnorm_apply_params(x, y, batch, spatial, channels, params, input_bias, act, slope, residual,
                        st);
}

// ---- allocation-free InstanceNorm + LeakyReLU ---------------------------------------
// `scratch` replaces the caller's workspace of instnorm_lrelu: per-chunk partials and the
// per-(b, c) parameters, instnorm_workspace_bytes() of it.  Every device the library runs on
// holds its own copy until the process ends.  Nothing in it needs clearing between calls
// (the statistics pass writes every partial the merge reads, the merge every parameter the
// apply pass reads), but two calls in flight on one device share it and race.
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of the current device's `scratch`, looked up on the first call on that
// device (the array's name is only a host-side handle, not a device address).
void* scratch_address() {
  int device = -1;
  hip_check(hipGetDevice(&device), "hipGetDevice");
  require(device >= 0 && device < kMaxScratchDevices, "device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* ptr = nullptr;
    hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    require(ptr != nullptr, "scratch symbol has no device address");
    g_scratch_ptr[device] = ptr;
  }
  return g_scratch_ptr[device];
}
}  // namespace

size_t instnorm_noalloc_max_bytes() { return kNoAllocScratchBytes; }

void instnorm_lrelu_noalloc(const float* x, float* y, int batch, int64_t spatial, int channels,
                            const float* input_bias, const float* gamma, const float* beta,
                            float eps, bool act, float slope, const float* residual,
                            hipStream_t st) {
  require(x && y, "instance normalisation pointers must not be null");
  require(batch >= 1 && spatial >= 1 && channels >= 1,
          "instance normalisation needs a non-empty tensor");
  const size_t need = instnorm_workspace_bytes(batch, spatial, channels);
  if (need > kNoAllocScratchBytes)
    fail(NNX_ERR_INVALID, "instance normalisation of this size needs " + std::to_string(need) +
                              " bytes of workspace, more than the allocation-free entry's " +
                              std::to_string(kNoAllocScratchBytes) +
                              "-byte scratch; use nnx_instnorm_lrelu with a workspace");
  instnorm_lrelu(x, y, batch, spatial, channels, input_bias, gamma, beta, eps, act, slope,
                 residual, scratch_address(), kNoAllocScratchBytes, st);
}

void instnorm_merge_partials(float4* partials, int nparts, int batch, int64_t spatial,
                             int channels, const float* gamma, const float* beta, float eps,
                             float4* params, hipStream_t st) {
  require(partials && params, "instance normalisation partials must not be null");
  require(nparts >= 1 && batch >= 1 && batch <= 65535 && channels >= 1 && channels <= 512,
          "invalid partial layout");
  ProfScope prof("instnorm_merge", 0.0, 16.0 * (double)batch * nparts * channels, st);
  const dim3 fgrid((unsigned)ceil_div(channels, 4), batch);  // a wave per (b, c)
  if (nparts <= 64) {
    hipLaunchKernelGGL(norm_merge_final_kernel, fgrid, dim3(256), 0, st, partials, params, beta,
                       gamma, spatial, channels, nparts, nparts, 1, eps);
    launch_check("instnorm merge partials");
    return;
  }
  // ~2048 blocks in all; nslices <= nparts / 2 balanced slices of at least two rows each (a
  // slice's result takes its first two rows)
  const int nslices = (int)std::max<int64_t>(1, std::min<int64_t>(ceil_div(2048, batch), nparts / 2));
  hipLaunchKernelGGL(norm_merge_slices_kernel, dim3(nslices, batch), dim3(256), 0, st, partials,
                     channels, nparts);
  launch_check("instnorm merge slices");
  hipLaunchKernelGGL(norm_merge_final_kernel, fgrid, dim3(256), 0, st, partials, params, beta,
                     gamma, spatial, channels, nparts, nslices, 0, eps);
  launch_check("instnorm merge partials");
}

void instnorm_apply_params(const float* x, float* y, int batch, int64_t spatial, int channels,
                           const float4* params, const float* input_bias, bool act, float slope,
                           const float* residual, hipStream_t st) {
  require(x && y && params, "instance normalisation pointers must not be null");
  require(channels >= 1 && channels <= 1024, "instance normalisation supports 1 to 1024 channels");
  require(batch >= 1 && batch <= 65535, "instance normalisation batch out of range");
  const int vw = channels % 4 == 0 ? 4 : 1;
  const double nelem = (double)batch * spatial * channels;
  ProfScope prof("instnorm_apply", 0.0, 4.0 * nelem * (residual ? 3 : 2), st);
  const int64_t sc = spatial * channels;
  const int64_t nvec = sc / vw;
  // blocks a batch item: one run of 1024 vectors each, up to 16384 (then they loop)
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(ceil_div(nvec, 1024), 16384));
  const size_t smem = (size_t)channels * 4 * sizeof(float);
  if (vw == 4)
    hipLaunchKernelGGL(norm_apply_kernel<4>, dim3((unsigned)blocks, batch), dim3(256), smem, st,
                       x, y, params, input_bias, residual, sc, channels, act ? 1 : 0, slope);
  else
    hipLaunchKernelGGL(norm_apply_kernel<1>, dim3((unsigned)blocks, batch), dim3(256), smem, st,
                       x, y, params, input_bias, residual, sc, channels, act ? 1 : 0, slope);
  launch_check("instnorm apply");
}

void avgpool3d(const float* x, float* y, int batch, const int* in_size, int channels,
               const int* kernel, hipStream_t st) {
  require(x && y, "pooling pointers must not be null");
  for (int i = 0; i < 3; ++i)
    require(kernel[i] >= 1 && in_size[i] >= kernel[i], "invalid pooling geometry");
  const int od = in_size[0] / kernel[0], oh = in_size[1] / kernel[1], ow = in_size[2] / kernel[2];
  const int64_t nout = (int64_t)batch * od * oh * ow * channels;
  require((int64_t)batch * od <= 65535 && oh <= 65535, "pooling output too large for the grid");
  const int vw = channels % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(y) % 16 == 0
                     ? 4
                     : 1;
  const dim3 grid((unsigned)ceil_div((int64_t)ow * (channels / vw), 256), (unsigned)oh,
                  (unsigned)(batch * od));
  ProfScope prof("avgpool3d", 0.0, 4.0 * (double)nout * (1 + kernel[0] * kernel[1] * kernel[2]), st);
  if (vw == 4)
    hipLaunchKernelGGL(avgpool_kernel<4>, grid, dim3(256), 0, st, x, y, in_size[0], in_size[1],
                       in_size[2], channels, kernel[0], kernel[1], kernel[2]);
  else
    hipLaunchKernelGGL(avgpool_kernel<1>, grid, dim3(256), 0, st, x, y, in_size[0], in_size[1],
                       in_size[2], channels, kernel[0], kernel[1], kernel[2]);
  launch_check("avgpool3d");
}

void match_spatial(const float* x, const int* in_size, float* y, const int* out_size, int batch,
                   int channels, hipStream_t st) {
  require(x && y && x != y, "crop/pad needs distinct input and output buffers");
  int off[3];
  for (int i = 0; i < 3; ++i) {
    require(in_size[i] >= 1 && out_size[i] >= 1, "crop/pad sizes must be positive");
    off[i] = (in_size[i] - out_size[i]) / 2;
  }
  const int vw = channels % 4 == 0 ? 4 : 1;
  const int64_t nout = (int64_t)batch * out_size[0] * out_size[1] * out_size[2] * (channels / vw);
  const int64_t blocks = std::min<int64_t>(ceil_div(nout, 256), 65536);
  ProfScope prof("match_spatial", 0.0, 8.0 * (double)nout * vw, st);
  if (vw == 4)
    hipLaunchKernelGGL(match_spatial_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, st, x, y,
                       nout, in_size[0], in_size[1], in_size[2], out_size[0], out_size[1],
                       out_size[2], channels, off[0], off[1], off[2]);
  else
    hipLaunchKernelGGL(match_spatial_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, st, x, y,
                       nout, in_size[0], in_size[1], in_size[2], out_size[0], out_size[1],
                       out_size[2], channels, off[0], off[1], off[2]);
  launch_check("match_spatial");
}

void count_nonfinite(const float* x, int64_t n, unsigned int* count, hipStream_t st) {
  require(count != nullptr, "count pointer must not be null");
  fill_zero(count, sizeof(unsigned int), st);
  if (n <= 0) return;
  require(x != nullptr, "input pointer must not be null");
  const int64_t blocks = std::min<int64_t>(ceil_div(n, 256), 4096);
  hipLaunchKernelGGL(nonfinite_kernel, dim3((unsigned)blocks), dim3(256), 0, st, x, n, count);
  launch_check("count_nonfinite");
}

void fill_zero(void* ptr, size_t bytes, hipStream_t st) {
  if (bytes == 0) return;
  require(ptr != nullptr, "fill pointer must not be null");
  if (bytes % 4 == 0 && reinterpret_cast<uintptr_t>(ptr) % 4 == 0) {
    const int64_t n = (int64_t)(bytes / 4);
    const int64_t blocks = std::min<int64_t>(ceil_div(n, 256), 65536);
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                       reinterpret_cast<uint32_t*>(ptr), n);
  } else {
    const int64_t n = (int64_t)bytes;
    const int64_t blocks = std::min<int64_t>(ceil_div(n, 256), 65536);
    hipLaunchKernelGGL(fill_zero_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                       reinterpret_cast<unsigned char*>(ptr), n);
  }
  launch_check("fill_zero");
}

}  // namespace nnx
