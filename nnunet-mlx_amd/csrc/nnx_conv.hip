// Convolutions of the nnU-Net forward on gfx950:
//   * conv3d_igemm  — implicit GEMM on v_mfma_f32_16x16x4_f32 with LDS-staged halo tiles
//                     (3^3 and any odd kernel, stride 1/2, two-pointer concat input)
//   * direct_cin1   — one-input-channel 3^3 convolution (K = 27 is too small for MFMA)
//   * pw_gemm       — pointwise GEMM on MFMA: stride==kernel ConvTranspose3d with the
//                     interleaving done by the epilogue's store addresses
//   * conv1x1_valu  — segmentation head (few output classes, bandwidth bound)
//
// GEMM view of a convolution: M = output voxels, N = C_out, K = taps * C_in.
// MFMA 16x16x4 f32 operand layout (one wave, 64 lanes):
//   A (16x4): lane l supplies A[l % 16][l / 16]
//   B (4x16): lane l supplies B[l / 16][l % 16]
//   D (16x16): lane l holds D[4 * (l / 16) + r][l % 16] in accumulator register r
// K is walked in chunks of 8 input channels; inside a chunk and tap, lane slot s = l / 16
// owns channels 2s and 2s+1, consumed by two MFMA k-steps, so every lane reads one
// float2 of A from LDS and one float2 of B (weights) from global memory per tap.
#include <string>

#include "nnx_internal.h"

namespace nnx {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

constexpr int kChunk = 8;  // input channels per LDS halo chunk / packed weight chunk

__device__ __forceinline__ f4 mfma16x16x4(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------------
// Packed weight layout shared by the implicit GEMM and the pointwise GEMM:
//   packed[((chunk * taps + tap) * nblk + nb) * 64 + lane] = float2 {
//       W[n][tap][cin(chunk, 2*(lane/16) + 0)], W[n][tap][cin(chunk, 2*(lane/16) + 1)] }
//   with n = nb * 16 + lane % 16, zero where n >= C_out or the channel is padding.
// For a two-part (concat) input, chunks 0 .. chunks0-1 cover part 1 and the rest part 2,
// each part padded to a multiple of 8 channels; the weight's input-channel axis holds
// part 1 first (the upsampled tensor), then part 2 (the skip), as in concat((up, skip)).
// ---------------------------------------------------------------------------------
__global__ void pack_conv_weight_kernel(const float* __restrict__ w, f2* __restrict__ out,
                                        int cout, int taps, int c1, int c2, int chunks1,
                                        int chunks, int nblk) {
  const int64_t total = (int64_t)chunks * taps * nblk * 64;
  const int ctot = c1 + c2;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(i % 64);
    int64_t r = i / 64;
    const int nb = (int)(r % nblk);
    r /= nblk;
    const int tap = (int)(r % taps);
    const int chunk = (int)(r / taps);
    const int n = nb * 16 + (lane & 15);
    f2 v = {0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int q = 2 * (lane >> 4) + e;
      int cin;
      bool ok;
      if (chunk < chunks1) {
        cin = chunk * kChunk + q;
        ok = cin < c1;
      } else {
        const int local = (chunk - chunks1) * kChunk + q;
        ok = local < c2;
        cin = c1 + local;
      }
      if (ok && n < cout) v[e] = w[((int64_t)n * taps + tap) * ctot + cin];
    }
    out[i] = v;
  }
}

// Pointwise (K = C_in) packing for the transposed convolution: column n enumerates
// (kd, kh, kw, o) with o fastest, so a 16-column block stores 16 consecutive channels.
__global__ void pack_tconv_weight_kernel(const float* __restrict__ w, f2* __restrict__ out,
                                         int cout, int koff, int cin, int chunks, int nblk) {
  const int64_t total = (int64_t)chunks * nblk * 64;
  const int ncols = koff * cout;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(i % 64);
    const int64_t r = i / 64;
    const int nb = (int)(r % nblk);
    const int chunk = (int)(r / nblk);
    const int n = nb * 16 + (lane & 15);
    f2 v = {0.f, 0.f};
    if (n < ncols) {
      const int o = n % cout;
      const int off = n / cout;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int c = chunk * kChunk + 2 * (lane >> 4) + e;
        // reference layout (C_out, kD, kH, kW, C_in): offset index enumerates (kd, kh, kw)
        if (c < cin) v[e] = w[((int64_t)o * koff + off) * cin + c];
      }
    }
    out[i] = v;
  }
}

// ---------------------------------------------------------------------------------
// Implicit GEMM with LDS halo tiles.
// One workgroup computes an output box bz x by x bx (one batch item) for WN*NB*16
// output channels.  Waves are arranged WM x WN; wave (wm, wn) owns MB row blocks of 16
// box voxels (box order, x fastest) and NB column blocks of 16 channels.
// For each 8-channel chunk the input halo ((b-1)*s + k per axis) is staged in LDS as
// [hz][hy][hx][8] floats; every tap then reads its A fragments from LDS.
// ---------------------------------------------------------------------------------
struct IgemmArgs {
  const float* x0;
  const float* x1;
  int c0, c1, chunks0, chunks;
  const f2* w;
  const float* bias;
  float* y;
  int id, ih, iw;
  int od, oh, ow;
  int cout, nblk;
  int kd, kh, kw, taps;
  int sd, sh, sw, pd, ph, pw;
  int bz, by, bx;
  int hz, hy, hx;
  int tz, ty, tx;
  int ntn, nwg;
};

template <int MB, int NB, int WM, int WN>
__global__ __launch_bounds__(64 * WM* WN) void igemm_kernel(IgemmArgs a) {
  extern __shared__ __align__(16) float lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM;
  const int wn = wave / WM;
  const int logical = xcd_remap(blockIdx.x, a.nwg);
  const int nt = logical % a.ntn;
  int tile = logical / a.ntn;
  const int txi = tile % a.tx;
  tile /= a.tx;
  const int tyi = tile % a.ty;
  tile /= a.ty;
  const int tzi = tile % a.tz;
  const int b = tile / a.tz;
  const int oz0 = tzi * a.bz, oy0 = tyi * a.by, ox0 = txi * a.bx;
  const int iz0 = oz0 * a.sd - a.pd, iy0 = oy0 * a.sh - a.ph, ix0 = ox0 * a.sw - a.pw;

  const int row = lane & 15;
  const int slot = lane >> 4;
  int hbase[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int v = 16 * (wm * MB + mb) + row;
    const int vx = v % a.bx;
    const int vy = (v / a.bx) % a.by;
    const int vz = v / (a.bx * a.by);
    hbase[mb] = ((vz * a.sd) * a.hy + vy * a.sh) * a.hx + vx * a.sw;
  }
  const int nbk0 = nt * (WN * NB) + wn * NB;

  f4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f4{0.f, 0.f, 0.f, 0.f};

  const int hyx = a.hy * a.hx;
  const int hvox = a.hz * hyx;
  const f2* lds2 = reinterpret_cast<const f2*>(lds);

  for (int chunk = 0; chunk < a.chunks; ++chunk) {
    const float* src;
    int C, cb;
    if (chunk < a.chunks0) {
      src = a.x0;
      C = a.c0;
      cb = chunk * kChunk;
    } else {
      src = a.x1;
      C = a.c1;
      cb = (chunk - a.chunks0) * kChunk;
    }
    __syncthreads();
    for (int i = tid; i < hvox * 2; i += blockDim.x) {
      const int v = i >> 1, h = i & 1;
      const int hz_ = v / hyx;
      const int rem = v - hz_ * hyx;
      const int hy_ = rem / a.hx;
      const int hx_ = rem - hy_ * a.hx;
      const int z = iz0 + hz_, yy = iy0 + hy_, xx = ix0 + hx_;
      f4 val = {0.f, 0.f, 0.f, 0.f};
      if ((unsigned)z < (unsigned)a.id && (unsigned)yy < (unsigned)a.ih &&
          (unsigned)xx < (unsigned)a.iw) {
        const int c = cb + h * 4;
        const int64_t off = ((((int64_t)b * a.id + z) * a.ih + yy) * a.iw + xx) * C + c;
        if ((C & 3) == 0) {
          if (c < C) val = *reinterpret_cast<const f4*>(src + off);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (c + q < C) val[q] = src[off + q];
        }
      }
      *reinterpret_cast<f4*>(lds + v * kChunk + h * 4) = val;
    }
    __syncthreads();
    const f2* wc = a.w + (int64_t)chunk * a.taps * a.nblk * 64 + lane;
    for (int kz = 0; kz < a.kd; ++kz) {
      for (int ky = 0; ky < a.kh; ++ky) {
        for (int kx = 0; kx < a.kw; ++kx) {
          const int tap = (kz * a.kh + ky) * a.kw + kx;
          const int toff = (kz * a.hy + ky) * a.hx + kx;
          f2 av[MB], bv[NB];
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) av[mb] = lds2[(hbase[mb] + toff) * 4 + slot];
          const f2* wt = wc + ((int64_t)tap * a.nblk + nbk0) * 64;
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            bv[nb] = (nbk0 + nb < a.nblk) ? wt[nb * 64] : f2{0.f, 0.f};
#pragma unroll
          for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
              for (int nb = 0; nb < NB; ++nb)
                acc[mb][nb] = mfma16x16x4(av[mb][e], bv[nb][e], acc[mb][nb]);
        }
      }
    }
  }

  // Epilogue: D[4*slot + r][row] of block (mb, nb) -> voxel 16*(wm*MB+mb) + 4*slot + r,
  // channel (nbk0+nb)*16 + row; the bias is added as a separate float32 addition.
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int v = 16 * (wm * MB + mb) + 4 * slot + r;
      const int vx = v % a.bx;
      const int vy = (v / a.bx) % a.by;
      const int vz = v / (a.bx * a.by);
      const int z = oz0 + vz, yy = oy0 + vy, xx = ox0 + vx;
      if (z < a.od && yy < a.oh && xx < a.ow) {
        const int64_t ob = ((((int64_t)b * a.od + z) * a.oh + yy) * a.ow + xx) * a.cout;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const int n = (nbk0 + nb) * 16 + row;
          if (n < a.cout) {
            float val = acc[mb][nb][r];
            if (a.bias) val = val + a.bias[n];
            a.y[ob + n] = val;
          }
        }
      }
    }
  }
}

struct Variant {
  int MB, NB, WM, WN;
  int m() const { return 16 * MB * WM; }
  int n() const { return 16 * NB * WN; }
};

constexpr Variant kVarA{8, 2, 4, 1};  // M 512, N 32
constexpr Variant kVarB{4, 4, 4, 1};  // M 256, N 64
constexpr Variant kVarC{4, 4, 2, 2};  // M 128, N 128
constexpr Variant kVarD{2, 4, 4, 1};  // M 128, N 64
constexpr Variant kVarE{2, 4, 2, 2};  // M 64,  N 128

constexpr int64_t kMaxHaloBytes = 64 * 1024;

struct Box {
  int z, y, x;
  int hz, hy, hx;
  int64_t tiles;
};

Box choose_box(const Variant& v, const ConvGeom& g) {
  const int m = v.m();
  Box best{};
  bool have = false;
  double best_score = 0;
  for (int bx : {16, 8, 4}) {
    if (m % bx) continue;
    const int rows = m / bx;
    for (int by = 1; by <= rows; by *= 2) {
      if (rows % by) continue;
      const int bz = rows / by;
      Box c;
      c.z = bz;
      c.y = by;
      c.x = bx;
      c.hz = (bz - 1) * g.s[0] + g.k[0];
      c.hy = (by - 1) * g.s[1] + g.k[1];
      c.hx = (bx - 1) * g.s[2] + g.k[2];
      const int64_t halo = (int64_t)c.hz * c.hy * c.hx;
      if (halo * kChunk * 4 > kMaxHaloBytes) continue;
      c.tiles = ceil_div(g.out[0], bz) * ceil_div(g.out[1], by) * ceil_div(g.out[2], bx);
      // MFMA rows actually computed (padding waste) dominate; halo traffic breaks ties.
      const double score = (double)c.tiles * m + 0.25 * (double)c.tiles * halo;
      if (!have || score < best_score) {
        best = c;
        best_score = score;
        have = true;
      }
    }
  }
  require(have, "convolution kernel too large for the LDS halo tile");
  return best;
}

template <int MB, int NB, int WM, int WN>
void launch_igemm(const IgemmArgs& a, int nwg, size_t lds_bytes, hipStream_t st, double flops,
                  double bytes) {
  static const std::string name = "conv3d_igemm_m" + std::to_string(16 * MB * WM) + "n" +
                                  std::to_string(16 * NB * WN);
  ProfScope prof(name.c_str(), flops, bytes, st);
  hipLaunchKernelGGL((igemm_kernel<MB, NB, WM, WN>), dim3(nwg), dim3(64 * WM * WN), lds_bytes,
                     st, a);
  launch_check("conv3d_igemm");
}

// ---------------------------------------------------------------------------------
// One-input-channel 3x3x3 convolution: one thread per output voxel keeps the 27 taps
// in registers (zeros in the padding) and starts every output channel from 0 with
// fma over the taps in (kd, kh, kw) order.  The optional bias is a separate addition.
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void direct_cin1_kernel(const float* __restrict__ x,
                                                          const float* __restrict__ w,
                                                          const float* __restrict__ bias,
                                                          float* __restrict__ y, int64_t nvox,
                                                          int D, int H, int W, int cout) {
  __shared__ float ws[27 * 64];
  __shared__ float bs[64];
  for (int i = threadIdx.x; i < 27 * cout; i += blockDim.x) ws[i] = w[i];
  for (int i = threadIdx.x; i < cout; i += blockDim.x) bs[i] = bias ? bias[i] : 0.f;
  __syncthreads();
  const int64_t vox = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (vox >= nvox) return;
  const int xx = (int)(vox % W);
  const int yy = (int)((vox / W) % H);
  const int zz = (int)((vox / ((int64_t)W * H)) % D);
  const int64_t plane = (vox / ((int64_t)W * H * D)) * D;
  float taps[27];
#pragma unroll
  for (int kd = 0; kd < 3; ++kd) {
    const int d = zz + kd - 1;
#pragma unroll
    for (int kh = 0; kh < 3; ++kh) {
      const int h = yy + kh - 1;
#pragma unroll
      for (int kw = 0; kw < 3; ++kw) {
        const int ww = xx + kw - 1;
        const bool inside = d >= 0 && d < D && h >= 0 && h < H && ww >= 0 && ww < W;
        taps[(kd * 3 + kh) * 3 + kw] = inside ? x[((plane + d) * H + h) * W + ww] : 0.f;
      }
    }
  }
  const bool has_bias = bias != nullptr;
  for (int c = 0; c < cout; c += 4) {
    f4 out;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float s = 0.f;
#pragma unroll
      for (int t = 0; t < 27; ++t) s = fmaf(taps[t], ws[(c + q) * 27 + t], s);
      out[q] = has_bias ? s + bs[c + q] : s;
    }
    *reinterpret_cast<f4*>(y + vox * cout + c) = out;
  }
}

// ---------------------------------------------------------------------------------
// Pointwise GEMM (A rows are whole channel vectors, K = C_in) for the stride==kernel
// transposed convolution.  Column n = ((az*KH + ay)*KW + ax)*C_out + o; the epilogue
// stores D[m][n] to output voxel (z*KD+az, y*KH+ay, x*KW+ax), channel o, + bias[o].
// A fragments are read straight from global memory (each 128-byte line is reused by
// four consecutive chunks through L1); weights are packed MFMA fragments.
// ---------------------------------------------------------------------------------
struct PwArgs {
  const float* x;
  int cin;
  int64_t M;
  const f2* w;
  int nblk, chunks;
  const float* bias;
  float* y;
  int cout;
  int kd, kh, kw;
  int id, ih, iw;
  int ntn, nwg;
};

template <int MB, int NB, int WM, int WN>
__global__ __launch_bounds__(64 * WM* WN) void pw_gemm_kernel(PwArgs a) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM;
  const int wn = wave / WM;
  const int logical = xcd_remap(blockIdx.x, a.nwg);
  const int nt = logical % a.ntn;
  const int64_t mt = logical / a.ntn;
  const int row = lane & 15;
  const int slot = lane >> 4;
  const int64_t m0 = mt * (16 * MB * WM) + (int64_t)wm * MB * 16;
  const float* arow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    int64_t m = m0 + mb * 16 + row;
    if (m >= a.M) m = a.M - 1;
    arow[mb] = a.x + m * a.cin + 2 * slot;
  }
  const int nbk0 = nt * (WN * NB) + wn * NB;
  f4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f4{0.f, 0.f, 0.f, 0.f};
  const f2* wl = a.w + nbk0 * 64 + lane;
  for (int chunk = 0; chunk < a.chunks; ++chunk) {
    const int k = chunk * kChunk + 2 * slot;
    f2 av[MB], bv[NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      av[mb] = (k < a.cin) ? *reinterpret_cast<const f2*>(arow[mb] + chunk * kChunk)
                           : f2{0.f, 0.f};
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      bv[nb] = (nbk0 + nb < a.nblk) ? wl[((int64_t)chunk * a.nblk + nb) * 64] : f2{0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          acc[mb][nb] = mfma16x16x4(av[mb][e], bv[nb][e], acc[mb][nb]);
  }
  const int ncols = a.kd * a.kh * a.kw * a.cout;
  const int od = a.id * a.kd, oh = a.ih * a.kh, ow = a.iw * a.kw;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t m = m0 + mb * 16 + 4 * slot + r;
      if (m >= a.M) continue;
      const int xx = (int)(m % a.iw);
      const int yy = (int)((m / a.iw) % a.ih);
      const int64_t zb = m / ((int64_t)a.iw * a.ih);  // b * id + z
      const int zz = (int)(zb % a.id);
      const int64_t bb = zb / a.id;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int n = (nbk0 + nb) * 16 + row;
        if (n >= ncols) continue;
        const int o = n % a.cout;
        const int off = n / a.cout;
        const int ax = off % a.kw;
        const int ay = (off / a.kw) % a.kh;
        const int az = off / (a.kw * a.kh);
        const int64_t ov =
            ((bb * od + (zz * a.kd + az)) * oh + (yy * a.kh + ay)) * (int64_t)ow + (xx * a.kw + ax);
        float val = acc[mb][nb][r];
        if (a.bias) val = val + a.bias[o];
        a.y[ov * a.cout + o] = val;
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// 1x1x1 convolution with few outputs (segmentation head): one thread per voxel, the
// weights in LDS; s = fma chain over input channels, then + bias.
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void conv1x1_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ w,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ y, int64_t nvox,
                                                      int cin, int cout) {
  extern __shared__ float ws[];  // cout * cin
  for (int i = threadIdx.x; i < cout * cin; i += blockDim.x) ws[i] = w[i];
  __syncthreads();
  const int64_t vox = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (vox >= nvox) return;
  const float* xr = x + vox * cin;
  for (int o = 0; o < cout; ++o) {
    float s = 0.f;
    const float* wr = ws + o * cin;
    if ((cin & 3) == 0) {
      for (int c = 0; c < cin; c += 4) {
        const f4 v = *reinterpret_cast<const f4*>(xr + c);
        s = fmaf(v[0], wr[c], s);
        s = fmaf(v[1], wr[c + 1], s);
        s = fmaf(v[2], wr[c + 2], s);
        s = fmaf(v[3], wr[c + 3], s);
      }
    } else {
      for (int c = 0; c < cin; ++c) s = fmaf(xr[c], wr[c], s);
    }
    y[vox * cout + o] = bias ? s + bias[o] : s;
  }
}

}  // namespace

// ===================================================================================
ConvGeom make_conv_geom(int batch, const int* in_size, const int* ksize, const int* stride) {
  ConvGeom g{};
  require(batch >= 1, "convolution batch must be positive");
  g.batch = batch;
  for (int i = 0; i < 3; ++i) {
    require(in_size[i] >= 1, "convolution input size must be positive");
    require(ksize[i] >= 1 && ksize[i] % 2 == 1, "only positive odd convolution kernels are supported");
    require(stride[i] >= 1, "convolution stride must be positive");
    g.in[i] = in_size[i];
    g.k[i] = ksize[i];
    g.s[i] = stride[i];
    g.p[i] = ksize[i] / 2;
    g.out[i] = (in_size[i] + 2 * g.p[i] - ksize[i]) / stride[i] + 1;
    require(g.out[i] >= 1, "convolution output would be empty");
  }
  return g;
}

int64_t conv_packed_floats(int cout, const int* ksize, int c1, int c2) {
  const int64_t taps = (int64_t)ksize[0] * ksize[1] * ksize[2];
  const int64_t chunks = ceil_div(c1, kChunk) + ceil_div(c2, kChunk);
  const int64_t nblk = ceil_div(cout, 16);
  return chunks * taps * nblk * 64 * 2;
}

void conv_pack_weight(const float* d_w, int cout, const int* ksize, int c1, int c2,
                      float* d_packed, hipStream_t st) {
  require(cout >= 1 && c1 >= 1 && c2 >= 0, "invalid convolution channel counts");
  const int taps = ksize[0] * ksize[1] * ksize[2];
  const int chunks1 = (int)ceil_div(c1, kChunk);
  const int chunks = chunks1 + (int)ceil_div(c2, kChunk);
  const int nblk = (int)ceil_div(cout, 16);
  const int64_t total = (int64_t)chunks * taps * nblk * 64;
  const int blocks = (int)std::min<int64_t>(ceil_div(total, 256), 65536);
  hipLaunchKernelGGL(pack_conv_weight_kernel, dim3(blocks), dim3(256), 0, st, d_w,
                     reinterpret_cast<f2*>(d_packed), cout, taps, c1, c2, chunks1, chunks, nblk);
  launch_check("conv3d_pack_weight");
}

void conv3d_igemm(const float* x1, int c1, const float* x2, int c2, const float* packed,
                  const float* bias, float* y, const ConvGeom& g, int cout, hipStream_t st) {
  require(x1 && y && packed, "convolution pointers must not be null");
  require(c1 >= 1 && (c2 == 0 || x2), "invalid convolution inputs");
  const bool stride1 = g.s[0] == 1 && g.s[1] == 1 && g.s[2] == 1;
  const int64_t vox = (int64_t)g.out[0] * g.out[1] * g.out[2];
  Variant v;
  if (cout <= 32)
    v = stride1 ? kVarA : kVarD;
  else if (cout <= 64)
    v = stride1 ? kVarB : kVarD;
  else
    v = (vox * g.batch <= 8192) ? kVarE : kVarC;
  const Box box = choose_box(v, g);
  IgemmArgs a{};
  a.x0 = x1;
  a.x1 = x2;
  a.c0 = c1;
  a.c1 = c2;
  a.chunks0 = (int)ceil_div(c1, kChunk);
  a.chunks = a.chunks0 + (int)ceil_div(c2, kChunk);
  a.w = reinterpret_cast<const f2*>(packed);
  a.bias = bias;
  a.y = y;
  a.id = g.in[0];
  a.ih = g.in[1];
  a.iw = g.in[2];
  a.od = g.out[0];
  a.oh = g.out[1];
  a.ow = g.out[2];
  a.cout = cout;
  a.nblk = (int)ceil_div(cout, 16);
  a.kd = g.k[0];
  a.kh = g.k[1];
  a.kw = g.k[2];
  a.taps = g.k[0] * g.k[1] * g.k[2];
  a.sd = g.s[0];
  a.sh = g.s[1];
  a.sw = g.s[2];
  a.pd = g.p[0];
  a.ph = g.p[1];
  a.pw = g.p[2];
  a.bz = box.z;
  a.by = box.y;
  a.bx = box.x;
  a.hz = box.hz;
  a.hy = box.hy;
  a.hx = box.hx;
  a.tz = (int)ceil_div(g.out[0], box.z);
  a.ty = (int)ceil_div(g.out[1], box.y);
  a.tx = (int)ceil_div(g.out[2], box.x);
  a.ntn = (int)ceil_div(cout, v.n());
  const int64_t nwg = (int64_t)g.batch * a.tz * a.ty * a.tx * a.ntn;
  require(nwg < (1LL << 31), "convolution grid too large");
  a.nwg = (int)nwg;
  const size_t lds = (size_t)box.hz * box.hy * box.hx * kChunk * sizeof(float);
  // Algorithmic work: 2*C_in*C_out*taps per output voxel; bytes: input, output, weights once.
  const double out_vox = (double)g.batch * vox;
  const double in_vox = (double)g.batch * g.in[0] * g.in[1] * g.in[2];
  const double flops = 2.0 * (c1 + c2) * cout * a.taps * out_vox;
  const double bytes = 4.0 * (in_vox * (c1 + c2) + out_vox * cout + (double)a.taps * (c1 + c2) * cout);
  if (v.MB == 8)
    launch_igemm<8, 2, 4, 1>(a, a.nwg, lds, st, flops, bytes);
  else if (v.MB == 4 && v.WN == 1)
    launch_igemm<4, 4, 4, 1>(a, a.nwg, lds, st, flops, bytes);
  else if (v.MB == 4)
    launch_igemm<4, 4, 2, 2>(a, a.nwg, lds, st, flops, bytes);
  else if (v.WN == 1)
    launch_igemm<2, 4, 4, 1>(a, a.nwg, lds, st, flops, bytes);
  else
    launch_igemm<2, 4, 2, 2>(a, a.nwg, lds, st, flops, bytes);
}

void conv3d_direct_cin1(const float* x, const float* w, const float* bias, float* y, int batch,
                        const int* size, int cout, hipStream_t st) {
  require(x && w && y, "convolution pointers must not be null");
  require(cout >= 4 && cout <= 64 && cout % 4 == 0,
          "one-channel direct convolution supports 4..64 outputs in steps of 4");
  const int64_t nvox = (int64_t)batch * size[0] * size[1] * size[2];
  require(nvox >= 1, "empty convolution input");
  ProfScope prof("conv3d_direct_cin1", 2.0 * 27 * cout * (double)nvox, 4.0 * (double)nvox * (1 + cout), st);
  hipLaunchKernelGGL(direct_cin1_kernel, dim3((unsigned)ceil_div(nvox, 256)), dim3(256), 0, st,
                     x, w, bias, y, nvox, size[0], size[1], size[2], cout);
  launch_check("conv3d_direct_small_cin");
}

int64_t tconv_packed_floats(int cout, const int* ksize, int cin) {
  const int64_t koff = (int64_t)ksize[0] * ksize[1] * ksize[2];
  return ceil_div(cin, kChunk) * ceil_div(koff * cout, 16) * 64 * 2;
}

void tconv_pack_weight(const float* d_w, int cout, const int* ksize, int cin, float* d_packed,
                       hipStream_t st) {
  require(cout >= 1 && cin >= 1, "invalid transposed-convolution channel counts");
  const int koff = ksize[0] * ksize[1] * ksize[2];
  const int chunks = (int)ceil_div(cin, kChunk);
  const int nblk = (int)ceil_div((int64_t)koff * cout, 16);
  const int64_t total = (int64_t)chunks * nblk * 64;
  const int blocks = (int)std::min<int64_t>(ceil_div(total, 256), 65536);
  hipLaunchKernelGGL(pack_tconv_weight_kernel, dim3(blocks), dim3(256), 0, st, d_w,
                     reinterpret_cast<f2*>(d_packed), cout, koff, cin, chunks, nblk);
  launch_check("tconv3d_pack_weight");
}

void tconv3d_gemm(const float* x, int cin, const float* packed, const float* bias, float* y,
                  int batch, const int* in_size, int cout, const int* ksize, hipStream_t st) {
  require(x && packed && y, "transposed-convolution pointers must not be null");
  require(cin >= 2 && cin % 2 == 0, "transposed convolution needs an even channel count");
  for (int i = 0; i < 3; ++i) require(ksize[i] >= 1 && in_size[i] >= 1, "invalid tconv geometry");
  PwArgs a{};
  a.x = x;
  a.cin = cin;
  a.M = (int64_t)batch * in_size[0] * in_size[1] * in_size[2];
  a.w = reinterpret_cast<const f2*>(packed);
  a.chunks = (int)ceil_div(cin, kChunk);
  const int ncols = ksize[0] * ksize[1] * ksize[2] * cout;
  a.nblk = (int)ceil_div(ncols, 16);
  a.bias = bias;
  a.y = y;
  a.cout = cout;
  a.kd = ksize[0];
  a.kh = ksize[1];
  a.kw = ksize[2];
  a.id = in_size[0];
  a.ih = in_size[1];
  a.iw = in_size[2];
  constexpr int MB = 4, NB = 4, WM = 2, WN = 2;
  a.ntn = (int)ceil_div(ncols, 16 * NB * WN);
  const int64_t nwg = ceil_div(a.M, 16 * MB * WM) * a.ntn;
  require(nwg < (1LL << 31), "transposed-convolution grid too large");
  a.nwg = (int)nwg;
  ProfScope prof("tconv3d_gemm", 2.0 * (double)a.M * cin * ncols,
                 4.0 * ((double)a.M * (cin + ncols) + (double)cin * ncols), st);
  hipLaunchKernelGGL((pw_gemm_kernel<MB, NB, WM, WN>), dim3(a.nwg), dim3(64 * WM * WN), 0, st, a);
  launch_check("tconv3d_gemm");
}

void conv1x1(const float* x, int cin, const float* w, const float* bias, float* y, int64_t voxels,
             int cout, hipStream_t st) {
  require(x && w && y, "1x1 convolution pointers must not be null");
  require(cin >= 1 && cout >= 1 && (int64_t)cin * cout <= 16384,
          "1x1 convolution weight too large for the head kernel");
  require(voxels >= 1, "empty 1x1 convolution input");
  ProfScope prof("conv1x1_head", 2.0 * (double)voxels * cin * cout, 4.0 * (double)voxels * (cin + cout), st);
  hipLaunchKernelGGL(conv1x1_kernel, dim3((unsigned)ceil_div(voxels, 256)), dim3(256),
                     (size_t)cin * cout * sizeof(float), st, x, w, bias, y, voxels, cin, cout);
  launch_check("conv1x1");
}

}  // namespace nnx
