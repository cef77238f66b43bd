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
#include <cmath>
#include <cstdlib>
#include <string>

#include "nnx_internal.h"

namespace nnx {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

constexpr int kChunk = 8;  // input channels per LDS halo chunk / packed weight chunk

// Workgroup barrier for LDS data only: waits for this wave's LDS (and scalar) operations,
// not for its global loads and stores, which __syncthreads' fence also waits for.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

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
  int lbx, lbxy;  // log2(bx), log2(bx*by): box dims are powers of two
  int hz, hy, hx;
  int tz, ty, tx;
  int ntn, nwg;
  float4* stats;  // optional per-tile InstanceNorm partials [b][tile][cout] (mean, M2, n, 0)
  int vstore;     // epilogue through LDS with 16-byte stores (every column block full)
  const uint4* w16;   // split-fp16 packed weights (x3 kernel)
  int ntg;            // tap groups of 4 (x3 kernel)
  float out_scale;    // 1 / weight scale (x3 kernel)
  // pending InstanceNorm (+ LeakyReLU) of input 0 / 1: (mean, scale, beta, 0) per (b, c)
  const float4* nrm0;
  const float4* nrm1;
  int act0, act1;
  float slope;
};

// The pending normalisation of one halo line (4 channels c..c+3 of the chunk's source):
// parameters of missing channels (c + q >= C) are zero, so their zero loads stay zero.
struct NormLine {
  float m[4], s[4], b[4];
  bool on, act;
};

__device__ __forceinline__ NormLine norm_line(const IgemmArgs& a, int chunk, int b, int C, int c) {
  NormLine nl;
  const bool first = chunk < a.chunks0;
  const float4* p = first ? a.nrm0 : a.nrm1;
  nl.on = p != nullptr;
  nl.act = (first ? a.act0 : a.act1) != 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (nl.on && c + q < C) v = p[(int64_t)b * C + c + q];
    nl.m[q] = v.x;
    nl.s[q] = v.y;
    nl.b[q] = v.z;
  }
  return nl;
}

// r = fma(x - mean, scale, beta), then max(slope * r, r): the operations of the InstanceNorm
// apply pass, so a fused load produces the same bits.
__device__ __forceinline__ f4 norm_apply4(f4 v, const NormLine& nl, float slope) {
  f4 r;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float t = fmaf(v[q] - nl.m[q], nl.s[q], nl.b[q]);
    if (nl.act) t = fmaxf(slope * t, t);
    r[q] = t;
  }
  return r;
}

// A zeroed 16-byte line: padding voxels of an asynchronously loaded halo read from here.
__device__ __align__(16) float g_zero_line[4];

// Decode halo float4 `f` of the current chunk into its global source (or the zero line).
struct HaloSource {
  const float* src;
  int C, cb;
};

__device__ __forceinline__ const float* halo_address(const IgemmArgs& a, const HaloSource& hs,
                                                     int f, int nf4, int b, int iz0, int iy0,
                                                     int ix0, int hyx) {
  const float* zero = g_zero_line;
  if (f >= nf4) return zero;
  const int v = f >> 1, h = f & 1;
  const int hz_ = v / hyx;
  const int rem = v - hz_ * hyx;
  const int hy_ = rem / a.hx;
  const int hx_ = rem - hy_ * a.hx;
  const int z = iz0 + hz_, yy = iy0 + hy_, xx = ix0 + hx_;
  if ((unsigned)z >= (unsigned)a.id || (unsigned)yy >= (unsigned)a.ih ||
      (unsigned)xx >= (unsigned)a.iw)
    return zero;
  return hs.src + ((((int64_t)b * a.id + z) * a.ih + yy) * a.iw + xx) * hs.C + hs.cb + h * 4;
}

__device__ __forceinline__ HaloSource halo_source(const IgemmArgs& a, int chunk) {
  if (chunk < a.chunks0) return HaloSource{a.x0, a.c0, chunk * kChunk};
  return HaloSource{a.x1, a.c1, (chunk - a.chunks0) * kChunk};
}

// Shared epilogue of the implicit-GEMM kernels.  acc holds D blocks: D[4*slot + r][row] of
// block (mb, nb) is voxel 16*(wm*MB+mb) + 4*slot + r of the box and channel
// (nbk0+nb)*16 + row.  Values are first multiplied by out_scale (a power of two undoing a
// weight scale, exact; skipped when 1), then the bias is added as a separate float32
// addition; optional fused InstanceNorm partials, then the stores.
// VST: with a.vstore set, the tile is transposed through LDS (rows padded by 4 floats) and
// written as whole 16-byte words per lane, each voxel's channel run contiguous
// kFull: the tile lies wholly inside the output volume (no per-voxel checks).
template <int MB, int NB, int WM, int WN, bool VST, bool kFull>
__device__ __forceinline__ void igemm_epilogue_t(const IgemmArgs& a, f4 (&acc)[MB][NB], float* lds,
                                                 int wm, int wn, int slot, int row, int nbk0,
                                                 int b, int tzi, int tyi, int txi, int oz0,
                                                 int oy0, int ox0, float out_scale) {
  if (out_scale != 1.0f) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = acc[mb][nb] * out_scale;
  }
  // The passes below stream over the accumulator blocks and recompute voxel validity, so the
  // epilogue needs fewer registers than the main loop (which sets the occupancy).
  float bias_n[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int n = (nbk0 + nb) * 16 + row;
    bias_n[nb] = (a.bias && n < a.cout) ? a.bias[n] : 0.f;
  }
  const bool has_bias = a.bias != nullptr;
  auto voxel_ok = [&](int mb, int r, int* z, int* yy, int* xx) {
    const int v = 16 * (wm * MB + mb) + 4 * slot + r;
    const int vx = v & (a.bx - 1);
    const int vy = (v >> a.lbx) & (a.by - 1);
    const int vz = v >> a.lbxy;
    *z = oz0 + vz;
    *yy = oy0 + vy;
    *xx = ox0 + vx;
    return kFull || (*z < a.od && *yy < a.oh && *xx < a.ow);
  };
  if (a.stats) {
    if constexpr (VST) {
      // InstanceNorm partials of this tile in one pass: per wave, sums of d = v - s and d^2
      // about a shift s (the wave's first voxel, finite), over the valid voxels; the WM
      // waves' (n, mean, M2) are then merged (Chan) through LDS.
      float4* red4 = reinterpret_cast<float4*>(lds);  // WM * 16 * NB * WN entries
      constexpr int NWG = 16 * NB * WN;
      float sd[NB], sq[NB], sh[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const float v0 = has_bias ? acc[0][nb][0] + bias_n[nb] : acc[0][nb][0];
        sh[nb] = __shfl(v0, row);  // lane `row` holds voxel 16 * wm * MB of column row
        sd[nb] = 0.f;
        sq[nb] = 0.f;
      }
      float nv = 0.f;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          int z, yy, xx;
          if (voxel_ok(mb, r, &z, &yy, &xx)) {
            nv += 1.f;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
              const float d = (has_bias ? acc[mb][nb][r] + bias_n[nb] : acc[mb][nb][r]) - sh[nb];
              sd[nb] += d;
              sq[nb] = fmaf(d, d, sq[nb]);
            }
          }
        }
      nv += __shfl_xor(nv, 16);
      nv += __shfl_xor(nv, 32);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        sd[nb] += __shfl_xor(sd[nb], 16);
        sd[nb] += __shfl_xor(sd[nb], 32);
        sq[nb] += __shfl_xor(sq[nb], 16);
        sq[nb] += __shfl_xor(sq[nb], 32);
      }
      __syncthreads();  // every wave is past its last halo and weight read
      if (slot == 0) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          red4[wm * NWG + (wn * NB + nb) * 16 + row] = make_float4(sd[nb], sq[nb], sh[nb], nv);
      }
      __syncthreads();
      if (wm == 0 && slot == 0) {
        const int tile_s = (tzi * a.ty + tyi) * a.tx + txi;
        const int spt = a.tz * a.ty * a.tx;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const int n = (nbk0 + nb) * 16 + row;
          float cnt = 0.f, mean = 0.f, m2 = 0.f;
          for (int w = 0; w < WM; ++w) {
            const float4 e = red4[w * NWG + (wn * NB + nb) * 16 + row];
            if (e.w > 0.f) {
              const float mw = e.z + e.x / e.w;
              const float m2w = fmaxf(e.y - e.x * (e.x / e.w), 0.f);
              const float tot = cnt + e.w;
              const float delta = mw - mean;
              mean += delta * (e.w / tot);
              m2 += m2w + delta * delta * (cnt * e.w / tot);
              cnt = tot;
            }
          }
          if (n < a.cout)
            a.stats[((int64_t)b * spt + tile_s) * a.cout + n] = make_float4(mean, m2, cnt, 0.f);
        }
      }
    } else {
      // InstanceNorm partials of this tile, two-pass over the registers: the tile mean of
      // every channel (lane sums, xor-shuffles over the 4 row slots, then the WM waves
      // through LDS), then the centred sum of squares about it.
      constexpr int NWG = 16 * NB * WN;
      float* red = lds;  // WM * NWG floats; the halo is no longer read
      const float cnt = (float)((a.od - oz0 < a.bz ? a.od - oz0 : a.bz) *
                                (a.oh - oy0 < a.by ? a.oh - oy0 : a.by) *
                                (a.ow - ox0 < a.bx ? a.ow - ox0 : a.bx));
      float part[NB], mean[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) part[nb] = 0.f;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          int z, yy, xx;
          if (voxel_ok(mb, r, &z, &yy, &xx)) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
              part[nb] += has_bias ? acc[mb][nb][r] + bias_n[nb] : acc[mb][nb][r];
          }
        }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        part[nb] += __shfl_xor(part[nb], 16);
        part[nb] += __shfl_xor(part[nb], 32);
      }
      __syncthreads();
      if (slot == 0) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) red[wm * NWG + (wn * NB + nb) * 16 + row] = part[nb];
      }
      __syncthreads();
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        float t = 0.f;
        for (int w = 0; w < WM; ++w) t += red[w * NWG + (wn * NB + nb) * 16 + row];
        mean[nb] = t / cnt;
        part[nb] = 0.f;
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          int z, yy, xx;
          if (voxel_ok(mb, r, &z, &yy, &xx)) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
              const float v = has_bias ? acc[mb][nb][r] + bias_n[nb] : acc[mb][nb][r];
              const float d = v - mean[nb];
              part[nb] = fmaf(d, d, part[nb]);
            }
          }
        }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        part[nb] += __shfl_xor(part[nb], 16);
        part[nb] += __shfl_xor(part[nb], 32);
      }
      __syncthreads();
      if (slot == 0) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) red[wm * NWG + (wn * NB + nb) * 16 + row] = part[nb];
      }
      __syncthreads();
      if (wm == 0 && slot == 0) {
        const int tile_s = (tzi * a.ty + tyi) * a.tx + txi;
        const int spt = a.tz * a.ty * a.tx;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const int n = (nbk0 + nb) * 16 + row;
          float t = 0.f;
          for (int w = 0; w < WM; ++w) t += red[w * NWG + (wn * NB + nb) * 16 + row];
          if (n < a.cout)
            a.stats[((int64_t)b * spt + tile_s) * a.cout + n] = make_float4(mean[nb], t, cnt, 0.f);
        }
      }
    }
  }
  if constexpr (VST) {
    if (a.vstore) {
      constexpr int NCOL = 16 * NB * WN;
      constexpr int LDW = NCOL + 4;
      constexpr int MT = 16 * MB * WM;
      constexpr int NT = 64 * WM * WN;
      constexpr int Q = NCOL / 4;
      float* tile_out = lds;
      __syncthreads();  // every wave is past its last halo, weight and partial-sum read
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int v = 16 * (wm * MB + mb) + 4 * slot + r;
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            tile_out[v * LDW + (wn * NB + nb) * 16 + row] =
                has_bias ? acc[mb][nb][r] + bias_n[nb] : acc[mb][nb][r];
        }
      __syncthreads();
      const int n0 = (nbk0 - wn * NB) * 16;
      for (int i = threadIdx.x; i < MT * Q; i += NT) {
        const int v = i / Q, q = i - v * Q;
        const int z = oz0 + (v >> a.lbxy), yy = oy0 + ((v >> a.lbx) & (a.by - 1)),
                  xx = ox0 + (v & (a.bx - 1));
        if (z < a.od && yy < a.oh && xx < a.ow)
          *reinterpret_cast<f4*>(a.y + ((((int64_t)b * a.od + z) * a.oh + yy) * a.ow + xx) * a.cout +
                                 n0 + 4 * q) = *reinterpret_cast<const f4*>(tile_out + v * LDW + 4 * q);
      }
      return;
    }
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int z, yy, xx;
      if (voxel_ok(mb, r, &z, &yy, &xx)) {
        float* yrow = a.y + ((((int64_t)b * a.od + z) * a.oh + yy) * a.ow + xx) * a.cout;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const int n = (nbk0 + nb) * 16 + row;
          if (n < a.cout) yrow[n] = has_bias ? acc[mb][nb][r] + bias_n[nb] : acc[mb][nb][r];
        }
      }
    }
  }
}

template <int MB, int NB, int WM, int WN, bool VST = false>
__device__ __forceinline__ void igemm_epilogue(const IgemmArgs& a, f4 (&acc)[MB][NB], float* lds,
                                               int wm, int wn, int slot, int row, int nbk0, int b,
                                               int tzi, int tyi, int txi, int oz0, int oy0, int ox0,
                                               float out_scale) {
  // uniform over the workgroup
  if (oz0 + a.bz <= a.od && oy0 + a.by <= a.oh && ox0 + a.bx <= a.ow)
    igemm_epilogue_t<MB, NB, WM, WN, VST, true>(a, acc, lds, wm, wn, slot, row, nbk0, b, tzi, tyi,
                                                txi, oz0, oy0, ox0, out_scale);
  else
    igemm_epilogue_t<MB, NB, WM, WN, VST, false>(a, acc, lds, wm, wn, slot, row, nbk0, b, tzi,
                                                 tyi, txi, oz0, oy0, ox0, out_scale);
}

// ASYNC: both inputs have channel counts that are multiples of 8, so every halo float4 is
// a whole aligned 16-byte line (or padding).  The halo is double-buffered in LDS and the
// next chunk is fetched with global_load_lds_dwordx4 (direct to LDS, no registers), one
// load per thread per tap, so the in-order vmcnt waits for the weight prefetch never
// wait on a whole halo.  Otherwise the halo goes through registers between barriers.
template <int MB, int NB, int WM, int WN, bool ASYNC>
__global__ __launch_bounds__(64 * WM* WN, 3) void igemm_kernel(IgemmArgs a) {
  extern __shared__ __align__(16) float lds[];
  constexpr int NT = 64 * WM * WN;
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
    const int vx = v & (a.bx - 1);
    const int vy = (v >> a.lbx) & (a.by - 1);
    const int vz = v >> a.lbxy;
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
  const int nf4 = hvox * 2;                 // float4 lines per chunk
  const int dpt = (nf4 + NT - 1) / NT;      // lines per thread
  const int buf_floats = dpt * NT * 4;      // one (padded) halo buffer
  // wave-uniform LDS base of this wave's lines in round j: (j*NT + wave*64) lines
  const int wave_line0 = __builtin_amdgcn_readfirstlane(wave * 64);

  if constexpr (ASYNC) {
    const HaloSource hs = halo_source(a, 0);
    for (int j = 0; j < dpt; ++j) {
      const float* g = halo_address(a, hs, j * NT + tid, nf4, b, iz0, iy0, ix0, hyx);
      __builtin_amdgcn_global_load_lds(
          g, (__attribute__((address_space(3))) void*)(lds + (j * NT + wave_line0) * 4), 16, 0, 0);
    }
  }

  for (int chunk = 0; chunk < a.chunks; ++chunk) {
    const float* cur = lds + (ASYNC ? (chunk & 1) * buf_floats : 0);
    if constexpr (ASYNC) {
      __builtin_amdgcn_s_waitcnt(0);  // this thread's halo lines have landed in LDS
      __syncthreads();                // ... and everyone's; the other buffer is free
    } else {
      const HaloSource hs = halo_source(a, chunk);
      // every line i = tid + k*NT of this thread is half (tid & 1) of its voxel
      const NormLine nl = norm_line(a, chunk, b, hs.C, hs.cb + (tid & 1) * 4);
      __syncthreads();
      for (int i = tid; i < nf4; i += NT) {
        const int v = i >> 1, h = i & 1;
        const int hz_ = v / hyx;
        const int rem = v - hz_ * hyx;
        const int hy_ = rem / a.hx;
        const int hx_ = rem - hy_ * a.hx;
        const int z = iz0 + hz_, yy = iy0 + hy_, xx = ix0 + hx_;
        f4 val = {0.f, 0.f, 0.f, 0.f};
        if ((unsigned)z < (unsigned)a.id && (unsigned)yy < (unsigned)a.ih &&
            (unsigned)xx < (unsigned)a.iw) {
          const int c = hs.cb + h * 4;
          const int64_t off = ((((int64_t)b * a.id + z) * a.ih + yy) * a.iw + xx) * hs.C + c;
          if ((hs.C & 3) == 0) {
            if (c < hs.C) val = *reinterpret_cast<const f4*>(hs.src + off);
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (c + q < hs.C) val[q] = hs.src[off + q];
          }
          if (nl.on) val = norm_apply4(val, nl, a.slope);
        }
        *reinterpret_cast<f4*>(lds + v * kChunk + h * 4) = val;
      }
      __syncthreads();
    }
    const f2* lds2 = reinterpret_cast<const f2*>(cur);
    const bool prefetch = ASYNC && chunk + 1 < a.chunks;
    const HaloSource next_hs = halo_source(a, chunk + 1 < a.chunks ? chunk + 1 : chunk);
    float* next_buf = lds + (((chunk + 1) & 1) * buf_floats);

    // Taps are walked in (kz, ky, kx) order with the next tap's A (LDS) and B (weights)
    // fragments requested before the current tap's MFMAs, so their latency overlaps
    // the 2*MB*NB matrix instructions.  The packed weights hold whole column groups,
    // so the B loads need no guard.
    const f2* wc = a.w + (int64_t)chunk * a.taps * a.nblk * 64 + nbk0 * 64 + lane;
    const int tap_stride = a.nblk * 64;
    f2 av[MB], bv[NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) av[mb] = lds2[hbase[mb] * 4 + slot];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) bv[nb] = wc[nb * 64];
    int kx = 0, ky = 0, kz = 0;
    for (int tap = 0; tap < a.taps; ++tap) {
      if (tap + 1 < a.taps) {
        if (++kx == a.kw) {
          kx = 0;
          if (++ky == a.kh) {
            ky = 0;
            ++kz;
          }
        }
      }
      const int ntap = tap + 1 < a.taps ? tap + 1 : tap;
      const int ntoff = (kz * a.hy + ky) * a.hx + kx;
      f2 an[MB], bn[NB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) an[mb] = lds2[(hbase[mb] + ntoff) * 4 + slot];
      const f2* wt = wc + (int64_t)ntap * tap_stride;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) bn[nb] = wt[nb * 64];
      if (prefetch && tap < dpt) {
        // round `tap` of the next chunk's halo lines, after this tap's weight loads;
        // rounds left over when dpt > taps are issued after the last tap
        const float* g = halo_address(a, next_hs, tap * NT + tid, nf4, b, iz0, iy0, ix0, hyx);
        __builtin_amdgcn_global_load_lds(
            g, (__attribute__((address_space(3))) void*)(next_buf + (tap * NT + wave_line0) * 4),
            16, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            acc[mb][nb] = mfma16x16x4(av[mb][e], bv[nb][e], acc[mb][nb]);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) av[mb] = an[mb];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) bv[nb] = bn[nb];
    }
    if (prefetch) {
      for (int j = a.taps; j < dpt; ++j) {
        const float* g = halo_address(a, next_hs, j * NT + tid, nf4, b, iz0, iy0, ix0, hyx);
        __builtin_amdgcn_global_load_lds(
            g, (__attribute__((address_space(3))) void*)(next_buf + (j * NT + wave_line0) * 4), 16,
            0, 0);
      }
    }
  }

  // (the checked epilogue only: a whole-tile copy beside it costs this kernel's registers)
  igemm_epilogue_t<MB, NB, WM, WN, false, false>(a, acc, lds, wm, wn, slot, row, nbk0, b, tzi, tyi,
                                                 txi, oz0, oy0, ox0, 1.0f);
}


// ---------------------------------------------------------------------------------
// "fp32-class" implicit GEMM on v_mfma_f32_16x16x32_f16.  Every float32 operand is split
// into fp16 halves x = hi + lo (hi = fp16(x), lo = fp16(x - hi), the difference being
// exact in float32); each product uses hi*hi + hi*lo + lo*hi (the lo*lo term, ~2^-22
// relative, is dropped) with float32 accumulation.  Weights are scaled by a power of two
// before splitting so their low halves stay normal; the epilogue multiplies by the
// inverse (exact).  One MFMA's K = 32 spans 4 taps x 8 channels: lane slot s = lane/16
// takes tap 4g + s of tap group g and channels 0..7 of the chunk, i.e. one 16-byte read
// from each of the two LDS planes (hi, lo: [halo voxel][8 halves]).  Taps beyond the
// kernel (the last group of 27 taps) read voxel 0 and meet zero weights.
// ---------------------------------------------------------------------------------
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f4 mfma16x16x32h(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void split_half(float v, _Float16& hi, _Float16& lo) {
  hi = (_Float16)v;
  lo = (_Float16)(v - (float)hi);
}

// Operand arithmetic of the split kernels.  kSplit3: fp16 hi/lo halves, three products
// hi*hi + hi*lo + lo*hi (float32 class).  kBf16: one bf16 operand per value (round to
// nearest even), one product; its bits travel in the same fp16-typed planes and words.
constexpr int kSplit3 = kArithSplit3;
constexpr int kBf16 = kArithBf16;
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f4 mfma16x16x32bf(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8, a),
                                                 __builtin_bit_cast(bf8, b), c, 0, 0, 0);
}

template <int AR>
__device__ __forceinline__ void to_operand(float v, _Float16& hi, _Float16& lo) {
  if constexpr (AR == kBf16) {
    hi = __builtin_bit_cast(_Float16, (__bf16)v);
    lo = (_Float16)0.f;
  } else {
    split_half(v, hi, lo);
  }
}

// to_operand of four values.  kSplit3: hi by v_cvt_pk_f16_f32 (nearest even, two values an
// instruction) and lo by one v_fma_mix{lo,hi}_f16 each: fma(hi, -1, v) is v - hi, exact in
// float32 (hi is v's nearest fp16), rounded once to fp16, i.e. the same bits as
// split_half's fp16(v - float(hi)) in 1.5 instructions a value instead of 4.
template <int AR>
__device__ __forceinline__ void to_operand4(const f4& v, h4& hv, h4& lv) {
  if constexpr (AR == kBf16) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      _Float16 hh, ll;
      to_operand<kBf16>(v[q], hh, ll);
      hv[q] = hh;
      lv[q] = ll;
    }
  } else {
#pragma unroll
    for (int q = 0; q < 4; q += 2) {
      const h2 h = __builtin_convertvector((f2{v[q], v[q + 1]}), h2);
      h2 l;
      asm("v_fma_mixlo_f16 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(l) : "v"(h), "v"(v[q]));
      asm("v_fma_mixhi_f16 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
          : "+v"(l) : "v"(h), "v"(v[q + 1]));
      hv[q] = h[0];
      hv[q + 1] = h[1];
      lv[q] = l[0];
      lv[q + 1] = l[1];
    }
  }
}

// acc[mb][nb] += A[mb] * B[nb] in the arithmetic AR; the passes touch MB*NB independent
// accumulators in turn (hi*hi, then hi*lo, then lo*hi for kSplit3).
template <int AR, int MB, int NB>
__device__ __forceinline__ void mma_products(f4 (&acc)[MB][NB], const h8 (&A)[MB][2],
                                             const h8 (&B)[NB][2]) {
  if constexpr (AR == kBf16) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = mfma16x16x32bf(A[mb][0], B[nb][0], acc[mb][nb]);
  } else {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = mfma16x16x32h(A[mb][0], B[nb][0], acc[mb][nb]);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = mfma16x16x32h(A[mb][0], B[nb][1], acc[mb][nb]);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = mfma16x16x32h(A[mb][1], B[nb][0], acc[mb][nb]);
  }
}

// Halo lines (8-byte halves of a voxel's 8-channel chunk, 4 floats) per thread: the
// split kernel stages the next chunk's halo in registers while the current chunk computes.
constexpr int kX3MaxLines = 6;  // halo lines per thread in flight (register staging)
constexpr int kX3Threads = 256;

// Weights stream one tap group ahead (double-buffered fragments).  Three workgroups share a
// CU: 150 registers with two column blocks a wave; with four the compiler fits 168 by
// spilling 4 registers outside the chunk loop (2.84 -> 2.60 ms a liver forward against two
// workgroups a CU at 182 registers).
template <int MB, int NB, int WM, int WN, int NTG, bool VEC, int AR>
__global__ __launch_bounds__(64 * WM* WN, 3) void igemm_x3_kernel(IgemmArgs a) {
  extern __shared__ __align__(16) float lds[];
  constexpr int NT = 64 * WM * WN;
  static_assert(NT == kX3Threads, "split kernel variants use 256 threads");
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
    const int vx = v & (a.bx - 1);
    const int vy = (v >> a.lbx) & (a.by - 1);
    const int vz = v >> a.lbxy;
    hbase[mb] = ((vz * a.sd) * a.hy + vy * a.sh) * a.hx + vx * a.sw;
  }
  const int nbk0 = nt * (WN * NB) + wn * NB;

  // halo offset of this lane's tap 4g + slot; padding taps (beyond the kernel) read voxel
  // 0 of the halo against zero weights
  int toff[NTG];
#pragma unroll
  for (int g = 0; g < NTG; ++g) {
    const int t = 4 * g + slot;
    int o = 0;
    if (t < a.taps) {
      const int kx = t % a.kw;
      const int r = t / a.kw;
      o = ((r / a.kh) * a.hy + r % a.kh) * a.hx + kx;
    }
    toff[g] = o;
  }

  f4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f4{0.f, 0.f, 0.f, 0.f};

  const int hyx = a.hy * a.hx;
  const int hvox = a.hz * hyx;
  const int nlines = hvox * 2;
  _Float16* hi_plane = reinterpret_cast<_Float16*>(lds);
  _Float16* lo_plane = hi_plane + (size_t)hvox * kChunk;
  const h8* hi8 = reinterpret_cast<const h8*>(hi_plane);
  const h8* lo8 = reinterpret_cast<const h8*>(lo_plane);

  // This thread's halo lines j*NT + tid: all share the half h = tid & 1 (NT is even); the
  // voxel index within the batch item is fixed across chunks (-1 outside the volume).
  const int h = tid & 1;
  int vofs[kX3MaxLines];
#pragma unroll
  for (int j = 0; j < kX3MaxLines; ++j) {
    const int line = j * NT + tid;
    int o = -1;
    if (line < nlines) {
      const int v = line >> 1;
      const int hz_ = v / hyx;
      const int rem = v - hz_ * hyx;
      const int hy_ = rem / a.hx;
      const int z = iz0 + hz_, yy = iy0 + hy_, xx = ix0 + (rem - hy_ * a.hx);
      if ((unsigned)z < (unsigned)a.id && (unsigned)yy < (unsigned)a.ih &&
          (unsigned)xx < (unsigned)a.iw)
        o = (z * a.ih + yy) * a.iw + xx;
    }
    vofs[j] = o;
  }
  const int64_t bvox = (int64_t)b * a.id * a.ih * a.iw;

  // The next chunk's lines are requested without branches (lines outside the volume read
  // a zero line) after the chunk's last weight request, so no weight wait (vector-memory
  // counters complete in issue order) queues behind them; they are used only at publish
  // time, where the pending normalisation is applied.
  const float* zero = g_zero_line;
  f4 stage[kX3MaxLines];
  NormLine nl_staged;
  auto fetch = [&](int chunk) {
    const HaloSource hs = halo_source(a, chunk);
    const int c = hs.cb + h * 4;
    nl_staged = norm_line(a, chunk, b, hs.C, c);
#pragma unroll
    for (int j = 0; j < kX3MaxLines; ++j) {
      if constexpr (VEC) {
        const float* src = vofs[j] >= 0 ? hs.src + (bvox + vofs[j]) * hs.C + c : zero;
        stage[j] = *reinterpret_cast<const f4*>(src);
      } else {
        f4 val = {0.f, 0.f, 0.f, 0.f};
        if (vofs[j] >= 0) {
          const int64_t off = (bvox + vofs[j]) * hs.C + c;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (c + q < hs.C) val[q] = hs.src[off + q];
        }
        stage[j] = val;
      }
    }
  };
  auto publish = [&]() {
#pragma unroll
    for (int j = 0; j < kX3MaxLines; ++j) {
      const int line = j * NT + tid;
      if (line < nlines) {
        f4 val = stage[j];
        if (nl_staged.on && vofs[j] >= 0) val = norm_apply4(val, nl_staged, a.slope);
        h4 hv, lv;
        to_operand4<AR>(val, hv, lv);
        *reinterpret_cast<h4*>(hi_plane + line * 4) = hv;
        if constexpr (AR == kSplit3) *reinterpret_cast<h4*>(lo_plane + line * 4) = lv;
      }
    }
  };

  fetch(0);
  const int group_stride = a.nblk * 128;
  for (int chunk = 0; chunk < a.chunks; ++chunk) {
    // packed weights: [chunk][group][nblk] x {hi h8 of 64 lanes, lo h8 of 64 lanes}
    const uint4* wc = a.w16 + ((int64_t)chunk * NTG * a.nblk + nbk0) * 128 + lane;
    h8 A[2][MB][2], B[2][NB][2];
    auto load_b = [&](int p, int g) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const uint4 wh = wc[g * group_stride + nb * 128];
        B[p][nb][0] = *reinterpret_cast<const h8*>(&wh);
        if constexpr (AR == kSplit3) {
          const uint4 wl = wc[g * group_stride + nb * 128 + 64];
          B[p][nb][1] = *reinterpret_cast<const h8*>(&wl);
        }
      }
    };
    auto load_a = [&](int p, int g) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        A[p][mb][0] = hi8[hbase[mb] + toff[g]];
        if constexpr (AR == kSplit3) A[p][mb][1] = lo8[hbase[mb] + toff[g]];
      }
    };
    load_b(0, 0);  // in flight across the barriers below
    __syncthreads();  // the previous chunk's fragments have been read
    publish();
    __syncthreads();
    load_a(0, 0);
#pragma unroll
    for (int g = 0; g < NTG; ++g) {
      const int cur = g & 1;
      if (g + 1 < NTG) {
        load_a(cur ^ 1, g + 1);
        load_b(cur ^ 1, g + 1);
      }
      mma_products<AR>(acc, A[cur], B[cur]);
    }
    if (chunk + 1 < a.chunks) fetch(chunk + 1);
  }
  igemm_epilogue<MB, NB, WM, WN>(a, acc, lds, wm, wn, slot, row, nbk0, b, tzi, tyi, txi, oz0, oy0,
                                 ox0, a.out_scale);
}

// Weight-staged split kernel: per chunk, the workgroup copies its halo (split into the
// two planes) and its weights (all NTG tap groups of its WN*NB column blocks) into LDS,
// then computes from LDS only.  The main loop issues no global loads, so its LDS waits
// never queue behind memory traffic; the chunk-boundary load latency is covered by the
// other resident workgroups.  LDS: 32 bytes per halo voxel + NTG * WN*NB * 2 KB.
template <int MB, int NB, int WM, int WN, int NTG, bool VEC, int AR>
__global__ __launch_bounds__(64 * WM* WN, 3) void igemm_x3s_kernel(IgemmArgs a) {
  extern __shared__ __align__(16) float lds[];
  constexpr int NT = 64 * WM * WN;
  constexpr int WBLK = WN * NB;  // column blocks of the workgroup
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
    const int vx = v & (a.bx - 1);
    const int vy = (v >> a.lbx) & (a.by - 1);
    const int vz = v >> a.lbxy;
    hbase[mb] = ((vz * a.sd) * a.hy + vy * a.sh) * a.hx + vx * a.sw;
  }
  const int nbk0 = nt * WBLK + wn * NB;

  int toff[NTG];
#pragma unroll
  for (int g = 0; g < NTG; ++g) {
    const int t = 4 * g + slot;
    int o = 0;
    if (t < a.taps) {
      const int kx = t % a.kw;
      const int r = t / a.kw;
      o = ((r / a.kh) * a.hy + r % a.kh) * a.hx + kx;
    }
    toff[g] = o;
  }

  f4 acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f4{0.f, 0.f, 0.f, 0.f};

  const int hyx = a.hy * a.hx;
  const int hvox = a.hz * hyx;
  const int nlines = hvox * 2;
  _Float16* hi_plane = reinterpret_cast<_Float16*>(lds);
  _Float16* lo_plane = hi_plane + (size_t)hvox * kChunk;
  const h8* hi8 = reinterpret_cast<const h8*>(hi_plane);
  const h8* lo8 = reinterpret_cast<const h8*>(lo_plane);
  // weights: [group][block][hi 64 lanes | lo 64 lanes] of 16 bytes
  uint4* wl = reinterpret_cast<uint4*>(lds + (size_t)hvox * 8);
  const h8* wl8 = reinterpret_cast<const h8*>(wl);

  const int h = tid & 1;  // every line j*NT + tid of this thread is half h of its voxel
  const int64_t bvox = (int64_t)b * a.id * a.ih * a.iw;
  const float* zero = g_zero_line;

  for (int chunk = 0; chunk < a.chunks; ++chunk) {
    const HaloSource hs = halo_source(a, chunk);
    const int c = hs.cb + h * 4;
    const NormLine nl = norm_line(a, chunk, b, hs.C, c);
    __syncthreads();  // the previous chunk's fragments have been read
    // halo: batches of kX3MaxLines loads in flight, then split + store
    for (int base = 0; base < nlines; base += kX3MaxLines * NT) {
      f4 val[kX3MaxLines];
      bool in[kX3MaxLines];
#pragma unroll
      for (int j = 0; j < kX3MaxLines; ++j) {
        const int line = base + j * NT + tid;
        const float* src = zero;
        bool inside = false;
        if (line < nlines) {
          const int v = line >> 1;
          const int hz_ = v / hyx;
          const int rem = v - hz_ * hyx;
          const int hy_ = rem / a.hx;
          const int z = iz0 + hz_, yy = iy0 + hy_, xx = ix0 + (rem - hy_ * a.hx);
          inside = (unsigned)z < (unsigned)a.id && (unsigned)yy < (unsigned)a.ih &&
                   (unsigned)xx < (unsigned)a.iw;
          if (inside) src = hs.src + (bvox + (int64_t)(z * a.ih + yy) * a.iw + xx) * hs.C + c;
        }
        in[j] = inside;
        if constexpr (VEC) {
          val[j] = *reinterpret_cast<const f4*>(src);
        } else {
          val[j] = f4{0.f, 0.f, 0.f, 0.f};
          if (inside) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (c + q < hs.C) val[j][q] = src[q];
          }
        }
      }
#pragma unroll
      for (int j = 0; j < kX3MaxLines; ++j) {
        const int line = base + j * NT + tid;
        if (line < nlines) {
          if (nl.on && in[j]) val[j] = norm_apply4(val[j], nl, a.slope);
          h4 hv, lv;
          to_operand4<AR>(val[j], hv, lv);
          *reinterpret_cast<h4*>(hi_plane + line * 4) = hv;
          if constexpr (AR == kSplit3) *reinterpret_cast<h4*>(lo_plane + line * 4) = lv;
        }
      }
    }
    // weights of this chunk and column range: NTG runs of WBLK*128 16-byte words
    {
      const uint4* wsrc = a.w16 + ((int64_t)chunk * NTG * a.nblk + nt * WBLK) * 128;
      constexpr int run = WBLK * 128;
      constexpr int total = NTG * run;
#pragma unroll
      for (int i0 = 0; i0 < total; i0 += NT) {
        const int i = i0 + tid;
        if (i < total) {
          const int g = i / run;
          wl[i] = wsrc[(int64_t)g * a.nblk * 128 + (i - g * run)];
        }
      }
    }
    __syncthreads();

    h8 A[2][MB][2], B[2][NB][2];
    auto load = [&](int p, int g) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        A[p][mb][0] = hi8[hbase[mb] + toff[g]];
        if constexpr (AR == kSplit3) A[p][mb][1] = lo8[hbase[mb] + toff[g]];
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int wb = (g * WBLK + wn * NB + nb) * 128 + lane;
        B[p][nb][0] = wl8[wb];
        if constexpr (AR == kSplit3) B[p][nb][1] = wl8[wb + 64];
      }
    };
    load(0, 0);
#pragma unroll
    for (int g = 0; g < NTG; ++g) {
      const int cur = g & 1;
      if (g + 1 < NTG) load(cur ^ 1, g + 1);
      mma_products<AR>(acc, A[cur], B[cur]);
    }
  }
  igemm_epilogue<MB, NB, WM, WN, true>(a, acc, lds, wm, wn, slot, row, nbk0, b, tzi, tyi, txi,
                                       oz0, oy0, ox0, a.out_scale);
}

// Split-fp16 weight packing: 16-byte words packed[((chunk * groups + g) * nblk + nb) * 128 +
// part * 64 + lane] = part 0: hi h8, part 1: lo h8 of scale * W[n][tap 4g + lane/16][cin(chunk,
// q)], q = 0..7, n = nb * 16 + lane % 16.
__global__ void pack_conv_weight_x3_kernel(const float* __restrict__ w, uint4* __restrict__ out,
                                           int cout, int taps, int c1, int c2, int chunks1,
                                           int chunks, int groups, int nblk, float scale,
                                           int arith) {
  const int64_t total = (int64_t)chunks * groups * nblk * 64;
  const int ctot = c1 + c2;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(i % 64);
    int64_t r = i / 64;
    const int nb = (int)(r % nblk);
    r /= nblk;
    const int g = (int)(r % groups);
    const int chunk = (int)(r / groups);
    const int n = nb * 16 + (lane & 15);
    const int tap = 4 * g + (lane >> 4);
    h8 hv, lv;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
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
      float v = 0.f;
      if (ok && n < cout && tap < taps) v = w[((int64_t)n * taps + tap) * ctot + cin] * scale;
      _Float16 hh, ll;
      if (arith == kBf16)
        to_operand<kBf16>(v, hh, ll);
      else
        to_operand<kSplit3>(v, hh, ll);
      hv[q] = hh;
      lv[q] = ll;
    }
    const int64_t word = (i - lane) * 2 + lane;  // block * 128 + lane
    out[word] = *reinterpret_cast<const uint4*>(&hv);
    out[word + 64] = *reinterpret_cast<const uint4*>(&lv);
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

// LDS budget per workgroup: one halo buffer of up to 64 KB (register path) or two of up
// to 32 KB each (asynchronous double-buffered path); lines are padded to whole rounds of
// the 256 threads.
constexpr int64_t kMaxLdsBytes = 64 * 1024;
constexpr int kThreads = 256;

struct Box {
  int z, y, x;
  int hz, hy, hx;
  int64_t tiles;
};

int64_t halo_buffer_bytes(int64_t halo_voxels) {
  return ceil_div(halo_voxels * 2, kThreads) * kThreads * 16;
}

Box choose_box(const Variant& v, const ConvGeom& g, bool double_buffer, int64_t max_halo = -1) {
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
      if (halo_buffer_bytes(halo) * (double_buffer ? 2 : 1) > kMaxLdsBytes) continue;
      if (max_halo >= 0 && halo > max_halo) continue;
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
void launch_igemm(const IgemmArgs& a, int nwg, bool async, hipStream_t st, double flops,
                  double bytes) {
  static const std::string name = "conv3d_igemm_m" + std::to_string(16 * MB * WM) + "n" +
                                  std::to_string(16 * NB * WN);
  constexpr int nt = 64 * WM * WN;
  const int64_t lines = (int64_t)a.hz * a.hy * a.hx * 2;
  const size_t buf_bytes = (size_t)ceil_div(lines, nt) * nt * 16;
  ProfScope prof(name.c_str(), flops, bytes, st);
  if (async)
    hipLaunchKernelGGL((igemm_kernel<MB, NB, WM, WN, true>), dim3(nwg), dim3(nt), 2 * buf_bytes,
                       st, a);
  else
    hipLaunchKernelGGL((igemm_kernel<MB, NB, WM, WN, false>), dim3(nwg), dim3(nt), buf_bytes, st,
                       a);
  launch_check("conv3d_igemm");
}

template <int MB, int NB, int WM, int WN, int NTG, bool VEC>
void launch_x3_vec(const IgemmArgs& a, int arith, size_t lds_bytes, hipStream_t st) {
  constexpr int nt = 64 * WM * WN;
  if (arith == kBf16)
    hipLaunchKernelGGL((igemm_x3_kernel<MB, NB, WM, WN, NTG, VEC, kBf16>), dim3(a.nwg), dim3(nt),
                       lds_bytes, st, a);
  else
    hipLaunchKernelGGL((igemm_x3_kernel<MB, NB, WM, WN, NTG, VEC, kSplit3>), dim3(a.nwg),
                       dim3(nt), lds_bytes, st, a);
}

template <int MB, int NB, int WM, int WN, int NTG>
void launch_x3_ntg(const IgemmArgs& a, bool vec, int arith, size_t lds_bytes, hipStream_t st) {
  if (vec)
    launch_x3_vec<MB, NB, WM, WN, NTG, true>(a, arith, lds_bytes, st);
  else
    launch_x3_vec<MB, NB, WM, WN, NTG, false>(a, arith, lds_bytes, st);
}

// Profiled kernel-class name of a split-kernel launch: "<base>_m<M>n<N>", with "_bf16"
// before the shape for the bf16 arithmetic.
std::string x3_launch_name(const char* base, int arith, int m, int n) {
  return std::string(base) + (arith == kBf16 ? "_bf16" : "") + "_m" + std::to_string(m) + "n" +
         std::to_string(n);
}

template <int MB, int NB, int WM, int WN>
void launch_x3(const IgemmArgs& a, bool vec, int arith, hipStream_t st, double flops,
               double bytes) {
  static const std::string names[2] = {
      x3_launch_name("conv3d_x3", kSplit3, 16 * MB * WM, 16 * NB * WN),
      x3_launch_name("conv3d_x3", kBf16, 16 * MB * WM, 16 * NB * WN)};
  // two fp16 planes of [halo voxel][8] = 32 bytes per halo voxel; the epilogue reuses
  // the first WM * 16 * NB * WN floats
  const size_t halo_bytes = (size_t)a.hz * a.hy * a.hx * 32;
  const size_t red_bytes = (size_t)WM * 16 * NB * WN * sizeof(float);
  const size_t lds_bytes = halo_bytes > red_bytes ? halo_bytes : red_bytes;
  ProfScope prof(names[arith == kBf16].c_str(), flops, bytes, st);
  if (a.ntg == 7)
    launch_x3_ntg<MB, NB, WM, WN, 7>(a, vec, arith, lds_bytes, st);
  else if (a.ntg == 3)
    launch_x3_ntg<MB, NB, WM, WN, 3>(a, vec, arith, lds_bytes, st);
  else
    launch_x3_ntg<MB, NB, WM, WN, 1>(a, vec, arith, lds_bytes, st);
  launch_check("conv3d_x3");
}

template <int MB, int NB, int WM, int WN, int NTG>
void launch_x3s_ntg(const IgemmArgs& a, bool vec, int arith, size_t lds_bytes, hipStream_t st) {
  constexpr int nt = 64 * WM * WN;
  if (arith == kBf16) {
    if (vec)
      hipLaunchKernelGGL((igemm_x3s_kernel<MB, NB, WM, WN, NTG, true, kBf16>), dim3(a.nwg),
                         dim3(nt), lds_bytes, st, a);
    else
      hipLaunchKernelGGL((igemm_x3s_kernel<MB, NB, WM, WN, NTG, false, kBf16>), dim3(a.nwg),
                         dim3(nt), lds_bytes, st, a);
  } else {
    if (vec)
      hipLaunchKernelGGL((igemm_x3s_kernel<MB, NB, WM, WN, NTG, true, kSplit3>), dim3(a.nwg),
                         dim3(nt), lds_bytes, st, a);
    else
      hipLaunchKernelGGL((igemm_x3s_kernel<MB, NB, WM, WN, NTG, false, kSplit3>), dim3(a.nwg),
                         dim3(nt), lds_bytes, st, a);
  }
}

size_t x3s_lds_bytes(int64_t halo_voxels, int ntg, int wblk) {
  return (size_t)halo_voxels * 32 + (size_t)ntg * wblk * 128 * 16;
}

template <int MB, int NB, int WM, int WN>
void launch_x3s(const IgemmArgs& a, bool vec, int arith, hipStream_t st, double flops,
                double bytes) {
  static const std::string names[2] = {
      x3_launch_name("conv3d_x3s", kSplit3, 16 * MB * WM, 16 * NB * WN),
      x3_launch_name("conv3d_x3s", kBf16, 16 * MB * WM, 16 * NB * WN)};
  const size_t red_bytes = (size_t)WM * 16 * NB * WN * sizeof(float);
  size_t lds_bytes = x3s_lds_bytes((int64_t)a.hz * a.hy * a.hx, a.ntg, WN * NB);
  if (lds_bytes < red_bytes) lds_bytes = red_bytes;
  if (a.vstore) {
    const size_t tile_bytes = (size_t)16 * MB * WM * (16 * NB * WN + 4) * sizeof(float);
    if (lds_bytes < tile_bytes) lds_bytes = tile_bytes;
  }
  ProfScope prof(names[arith == kBf16].c_str(), flops, bytes, st);
  if (a.ntg == 7)
    launch_x3s_ntg<MB, NB, WM, WN, 7>(a, vec, arith, lds_bytes, st);
  else if (a.ntg == 3)
    launch_x3s_ntg<MB, NB, WM, WN, 3>(a, vec, arith, lds_bytes, st);
  else
    launch_x3s_ntg<MB, NB, WM, WN, 1>(a, vec, arith, lds_bytes, st);
  launch_check("conv3d_x3s");
}

// ---------------------------------------------------------------------------------
// One-input-channel 3x3x3 convolution: one thread per output voxel takes its 27 taps
// (zeros in the padding) and starts every output channel from 0 with fma over the taps
// in (kd, kh, kw) order.  The optional bias is a separate addition.
// Grid: (4 x 8 x 8 tiles per batch item, batch); the tile's 6 x 10 x 10 input halo is read
// once into LDS.  Weights and bias are read through the constant address space: the
// loads are uniform, so they become scalar loads and every fma takes its weight from an
// SGPR.  The output rows are staged in LDS and leave as contiguous runs of 8 voxels.
// With `stats`, the tile also writes the InstanceNorm partials of its voxels,
// stats[(b * gridDim.x + tile) * cout + c] = (mean, M2, n, 0) of conv + bias, two-pass
// over the tile's outputs in LDS.
// ---------------------------------------------------------------------------------
constexpr int kDirTz = 4, kDirTy = 8, kDirTx = 8;
constexpr int kDirHz = kDirTz + 2, kDirHy = kDirTy + 2, kDirHx = kDirTx + 2;
// tile of the split-product kernel (256 voxels, x fastest)
constexpr int kDirX3Tz = 4, kDirX3Ty = 4, kDirX3Tx = 16;
constexpr int kDirX3TilesPerBlock = 16;

// the tile's 6 x 10 x 10 input halo (zeros outside the volume)
__device__ __forceinline__ void direct_stage_halo(float* halo, const float* __restrict__ x,
                                                  int64_t item, int D, int H, int W, int z0,
                                                  int y0, int x0) {
  for (int i = threadIdx.x; i < kDirHz * kDirHy * kDirHx; i += 256) {
    const int hz = i / (kDirHy * kDirHx), hy = (i / kDirHx) % kDirHy, hx = i % kDirHx;
    const int z = z0 + hz - 1, yy = y0 + hy - 1, xx = x0 + hx - 1;
    const bool inside = (unsigned)z < (unsigned)D && (unsigned)yy < (unsigned)H &&
                        (unsigned)xx < (unsigned)W;
    halo[i] = inside ? x[item + ((int64_t)z * H + yy) * W + xx] : 0.f;
  }
}

// Stores the tile's outputs (staged in out_s, rows of cout + 1 floats) as contiguous runs,
// then writes the tile's InstanceNorm partials when `stats` is set.  Call after a barrier
// that follows the out_s writes.
template <int COUT>
__device__ __forceinline__ void direct_store_tile(const float* out_s, float* red,
                                                  float* __restrict__ y, int64_t item, int D,
                                                  int H, int W, int z0, int y0, int x0,
                                                  float4* __restrict__ stats) {
  constexpr int cout = COUT;
  constexpr int stride = cout + 1;
  const int tid = threadIdx.x;
  // rows (tz, ty) of up to 8 voxels: cout * nx contiguous floats each, one wave per row
  const int nx = W - x0 < kDirTx ? W - x0 : kDirTx;
  const int wave = tid >> 6, lane = tid & 63;
  for (int r = wave; r < kDirTz * kDirTy; r += 4) {
    const int rz = r >> 3, ry = r & 7;
    if (z0 + rz >= D || y0 + ry >= H) continue;
    f4* dst = reinterpret_cast<f4*>(y + (item + ((int64_t)(z0 + rz) * H + y0 + ry) * W + x0) * cout);
    for (int i = lane; i < nx * cout / 4; i += 64) {
      const int e = i * 4;
      const int v = e / cout, c = e - v * cout;
      const float* src = out_s + (r * kDirTx + v) * stride + c;
      dst[i] = f4{src[0], src[1], src[2], src[3]};
    }
  }
  // statistics after the stores are issued, so they overlap the write-back
  if (stats) {
    // channel c = tid % cout over voxels part, part + parts, ...: tile mean, then centred M2
    const int nz = D - z0 < kDirTz ? D - z0 : kDirTz, ny = H - y0 < kDirTy ? H - y0 : kDirTy;
    const int nv = nz * ny * nx;
    const int parts = 256 / cout;
    const int c = tid % cout, part = tid / cout;
    const bool active = part < parts;
    auto in_tile = [&](int v) { return (v >> 6) < nz && ((v >> 3) & 7) < ny && (v & 7) < nx; };
    float t = 0.f;
    if (active)
      for (int v = part; v < 256; v += parts)
        if (in_tile(v)) t += out_s[v * stride + c];
    red[tid] = t;
    __syncthreads();
    float mean = 0.f;
    if (active) {
      for (int q = 0; q < parts; ++q) mean += red[q * cout + c];
      mean = mean / (float)nv;
    }
    __syncthreads();
    t = 0.f;
    if (active)
      for (int v = part; v < 256; v += parts)
        if (in_tile(v)) {
          const float d = out_s[v * stride + c] - mean;
          t = fmaf(d, d, t);
        }
    red[tid] = t;
    __syncthreads();
    if (part == 0) {
      float m2 = 0.f;
      for (int q = 0; q < parts; ++q) m2 += red[q * cout + c];
      stats[((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * cout + c] =
          make_float4(mean, m2, (float)nv, 0.f);
    }
  }
}

template <int COUT>
__global__ __launch_bounds__(256) void direct_cin1_kernel(const float* __restrict__ x,
                                                          const float* __restrict__ w,
                                                          const float* __restrict__ bias,
                                                          float* __restrict__ y, int D, int H,
                                                          int W, int tiles_y, int tiles_x,
                                                          float4* __restrict__ stats) {
  typedef const __attribute__((address_space(4))) float* cfloat_p;
  constexpr int cout = COUT;
  constexpr int stride = cout + 1;  // padded output rows: no bank conflicts
  __shared__ float halo[kDirHz * kDirHy * kDirHx];
  __shared__ float red[256];
  extern __shared__ float out_s[];  // 256 voxels x (cout + 1)
  const cfloat_p wc = (cfloat_p)w;
  const cfloat_p bc = (cfloat_p)bias;
  const int tid = threadIdx.x;
  const int tile = blockIdx.x;
  const int txi = tile % tiles_x, tyi = (tile / tiles_x) % tiles_y, tzi = tile / (tiles_x * tiles_y);
  const int z0 = tzi * kDirTz, y0 = tyi * kDirTy, x0 = txi * kDirTx;
  const int64_t item = (int64_t)blockIdx.y * D * H * W;  // first voxel of the batch item
  direct_stage_halo(halo, x, item, D, H, W, z0, y0, x0);
  __syncthreads();
  const int tz = tid >> 6, ty = (tid >> 3) & 7, tx = tid & 7;
  {
    float taps[27];
#pragma unroll
    for (int kd = 0; kd < 3; ++kd)
#pragma unroll
      for (int kh = 0; kh < 3; ++kh)
#pragma unroll
        for (int kw = 0; kw < 3; ++kw)
          taps[(kd * 3 + kh) * 3 + kw] = halo[((tz + kd) * kDirHy + ty + kh) * kDirHx + tx + kw];
    const bool has_bias = bias != nullptr;
#pragma unroll
    for (int c = 0; c < cout; ++c) {
      float sum = 0.f;
#pragma unroll
      for (int t = 0; t < 27; ++t) sum = fmaf(taps[t], wc[c * 27 + t], sum);
      out_s[tid * stride + c] = has_bias ? sum + bc[c] : sum;
    }
  }
  __syncthreads();
  direct_store_tile<COUT>(out_s, red, y, item, D, H, W, z0, y0, x0, stats);
}

// power of two that brings max |v| into [2^14, 2^15), at most 2^100 so that its inverse
// stays a normal float (1 for 0 or a non-finite maximum)
__device__ __forceinline__ float split_scale_of(float max_abs) {
  if (!(max_abs > 0.f) || !(max_abs <= 3.4e38f)) return 1.f;
  int e;
  frexpf(max_abs, &e);
  return ldexpf(1.f, 15 - e < 100 ? 15 - e : 100);
}

// Sum over the 16 lanes of each DPP row (row rotations by 8, 4, 2, 1); every lane of the
// row receives the sum.
template <int CTRL>
__device__ __forceinline__ float dpp_row(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp_row<0x128>(v);
  v += dpp_row<0x124>(v);
  v += dpp_row<0x122>(v);
  v += dpp_row<0x121>(v);
  return v;
}

// Waves a SIMD the first convolution is built for, where its registers fit without spills:
// 4 (at most 128 registers) for one input channel and at most 32 outputs, 2 (256) for four
// input channels and at most 48 outputs, else the compiler's choice.
template <int COUT, int CIN>
constexpr int kDirX3Waves = (CIN == 1 && COUT <= 32) ? 4 : (CIN == 4 && COUT <= 48) ? 2 : 1;

// The same convolution with split-fp16 products on MFMA for CIN = 1, 2 or 4 input
// channels: the weights of 16 output channels form 16 x 32 A fragments (27 * CIN (tap,
// channel) products zero-padded to whole K steps of 32), the taps of 16 voxels 32 x 16 B
// fragments, hi*hi + hi*lo + lo*hi with float32 accumulation.  The raw input
// has no normalised range, so each tile scales its halo by a power of two from the tile's
// own max |x| (weights by `wscale`, a power of two from max |w|) before the split and the
// products by the inverses (exact); + bias after.  Tiles of kDirX3Tz x kDirX3Ty x kDirX3Tx
// = 256 voxels (x fastest); wave w computes voxels 64 w .. 64 w + 63 of the tile:
// 4 blocks of 16 voxels x ceil(cout / 16) blocks of 16 channels.  A lane's accumulator
// holds 4 consecutive channels of one voxel, stored as one 16-byte word; the tile's
// InstanceNorm partials come from the accumulators in one pass (sums of x - s and its square,
// s a value of the wave's own first voxel, over the lanes of a DPP row; then per wave
// (count, mean, M2) merged across the 4 waves by Chan's formula), so the outputs never pass
// through LDS.  The halo is scaled and split once into fp16 hi/lo planes in LDS; barriers
// wait for LDS only, so output stores and the next tile's halo loads stay in flight.
template <int COUT, int CIN>
__global__ __launch_bounds__(256, (kDirX3Waves<COUT, CIN>)) void direct_cin1_x3_kernel(
    const float* __restrict__ x, const float* __restrict__ w, float wscale,
    const float* __restrict__ bias, float* __restrict__ y, int D, int H, int W, int tiles_y,
    int tiles_x, int ntiles, int tpb, float4* __restrict__ stats) {
  constexpr int cout = COUT;
  constexpr int NB = (COUT + 15) / 16;
  constexpr int MB = 4;
  constexpr int TZ = kDirX3Tz, TY = kDirX3Ty, TX = kDirX3Tx;
  constexpr int HY = TY + 2, HX = TX + 2;
  constexpr int kHalo = (TZ + 2) * HY * HX * CIN;  // voxel-major, CIN channels a voxel
  constexpr int K = 27 * CIN, KS = (K + 31) / 32;    // taps x channels, 32 per MFMA step
  constexpr int kLoads = (kHalo + 255) / 256;
  // the tile's scaled halo split once into fp16 hi and lo planes
  __shared__ __align__(16) _Float16 halo_hi[kHalo];
  __shared__ __align__(16) _Float16 halo_lo[kHalo];
  __shared__ float red[4][NB * 16], red2[4][NB * 16], wcnt[4];
  __shared__ float wmax[2][4];  // per-wave maxima of |x|, double-buffered over tiles
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int row = lane & 15, slot = lane >> 4;
  const int64_t item = (int64_t)blockIdx.y * D * H * W;
  const bool has_bias = bias != nullptr;

  // A fragments: lane (n = 16 nb + row, k = 32 s + 8 slot + q) holds wscale * W[n][k] split,
  // k = tap * CIN + channel (the (C_out, kD, kH, kW, C_in) layout), in registers, or with 4
  // channels (whose four K steps would not fit next to the accumulators) in LDS, read one K
  // step at a time; bias of the lane's 4 output channels 16 nb + 4 slot + r
  constexpr bool kALds = CIN > 2;
  __shared__ h8 a_lds[kALds ? NB * KS * 2 * 64 : 1];
  h8 A[kALds ? 1 : NB][kALds ? 1 : KS][2];
  f4 bn[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int n = nb * 16 + row;
#pragma unroll
    for (int st = 0; st < KS; ++st) {
      h8 fh, fl;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int k = st * 32 + slot * 8 + q;
        const float v = (n < cout && k < K) ? w[n * K + k] * wscale : 0.f;
        _Float16 hh, ll;
        to_operand<kSplit3>(v, hh, ll);
        fh[q] = hh;
        fl[q] = ll;
      }
      if constexpr (kALds) {
        a_lds[((nb * KS + st) * 2 + 0) * 64 + lane] = fh;
        a_lds[((nb * KS + st) * 2 + 1) * 64 + lane] = fl;
      } else {
        A[nb][st][0] = fh;
        A[nb][st][1] = fl;
      }
    }
    const int n0 = nb * 16 + slot * 4;
    bn[nb] = f4{0.f, 0.f, 0.f, 0.f};
    if (has_bias && n0 < cout) bn[nb] = f4{bias[n0], bias[n0 + 1], bias[n0 + 2], bias[n0 + 3]};
  }
  const float inv_w = 1.f / wscale;
  static_assert(TX == 16 && TY == 4, "a wave's voxels are one z-plane of the tile");
  // 4 channels: this lane's taps of K step st are 8 st + 2 slot + u (u = 0, 1); padded taps
  // (>= 27) read tap 0's voxel against zero weights
  int toff4[CIN == 4 ? KS : 1][2];
  if constexpr (CIN == 4) {
#pragma unroll
    for (int st = 0; st < KS; ++st)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int tap = 8 * st + 2 * slot + u;
        toff4[st][u] = tap < 27 ? ((tap / 9) * HY + (tap / 3) % 3) * HX + tap % 3 : 0;
      }
  }

  // tiles tpb * blockIdx.x .. of this batch item, one after the other; each tile's halo
  // is loaded into registers while the previous tile computes, and its maximum |x| is
  // reduced per wave at the end of the previous tile
  const int t_begin = blockIdx.x * tpb;
  const int t_end = min(ntiles, t_begin + tpb);
  float hv[kLoads];
  auto load_halo = [&](int tile) {
    const int txi = tile % tiles_x, tyi = (tile / tiles_x) % tiles_y, tzi = tile / (tiles_x * tiles_y);
    const int z0 = tzi * TZ, y0 = tyi * TY, x0 = txi * TX;
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const int i = tid + 256 * j;
      const int hvox = i / CIN, hc = i - hvox * CIN;
      const int hz = hvox / (HY * HX), hy = (hvox / HX) % HY, hx = hvox % HX;
      const int z = z0 + hz - 1, yy = y0 + hy - 1, xx = x0 + hx - 1;
      const bool inside = i < kHalo && (unsigned)z < (unsigned)D && (unsigned)yy < (unsigned)H &&
                          (unsigned)xx < (unsigned)W;
      hv[j] = inside ? x[(item + ((int64_t)z * H + yy) * W + xx) * CIN + hc] : 0.f;
    }
  };
  // maximum |x| over the registers' halo values (zeros outside the volume): per thread,
  // then per wave into wmax[buf]
  auto wave_max = [&](int buf) {
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < kLoads; ++j)
      if (tid + 256 * j < kHalo) mx = fmaxf(mx, fabsf(hv[j]));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (lane == 0) wmax[buf][wave] = mx;
  };
  if (t_begin < t_end) {
    load_halo(t_begin);
    wave_max(0);
  }
  for (int tile = t_begin; tile < t_end; ++tile) {
    const int buf = (tile - t_begin) & 1;
    const int txi = tile % tiles_x, tyi = (tile / tiles_x) % tiles_y, tzi = tile / (tiles_x * tiles_y);
    const int z0 = tzi * TZ, y0 = tyi * TY, x0 = txi * TX;
    // the previous tile's operand reads and partials are done; this tile's maxima are in
    // wmax[buf]
    lds_barrier();
    const float xscale =
        split_scale_of(fmaxf(fmaxf(wmax[buf][0], wmax[buf][1]), fmaxf(wmax[buf][2], wmax[buf][3])));
    // inverse scales, applied one after the other (exact powers of two; their product
    // alone could leave the float range)
    const float inv_x = 1.f / xscale;
    // publish the halo times xscale (exact) as fp16 hi and lo planes
#pragma unroll
    for (int j = 0; j < kLoads; ++j)
      if (tid + 256 * j < kHalo) {
        _Float16 hh, ll;
        to_operand<kSplit3>(hv[j] * xscale, hh, ll);
        halo_hi[tid + 256 * j] = hh;
        halo_lo[tid + 256 * j] = ll;
      }
    if (tile + 1 < t_end) load_halo(tile + 1);
    lds_barrier();

    f4 acc[MB][NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < KS; ++st) {
      h8 As[NB][2];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          if constexpr (kALds) As[nb][p] = a_lds[((nb * KS + st) * 2 + p) * 64 + lane];
          else As[nb][p] = A[nb][st][p];
        }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        // B fragment: lane (voxel v = 64 wave + 16 mb + row, taps 8 slot + q)
        // (a wave's 64 voxels are one z-plane of the tile: TY x TX = 4 x 16)
        const int base = (wave * HY + mb) * HX + row;
        h8 B[2];
        if constexpr (CIN == 4) {
          // two taps of 4 channels: one 8-byte read per tap and plane
          h4 th[2], tl[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            th[u] = *reinterpret_cast<const h4*>(halo_hi + (base + toff4[st][u]) * 4);
            tl[u] = *reinterpret_cast<const h4*>(halo_lo + (base + toff4[st][u]) * 4);
          }
          B[0] = __builtin_shufflevector(th[0], th[1], 0, 1, 2, 3, 4, 5, 6, 7);
          B[1] = __builtin_shufflevector(tl[0], tl[1], 0, 1, 2, 3, 4, 5, 6, 7);
        } else {
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const int k = st * 32 + slot * 8 + q;
            const int tap = k / CIN, hc = k - tap * CIN;
            const int off = k < K ? ((tap / 9) * HY + (tap / 3) % 3) * HX + tap % 3 : 0;
            B[0][q] = k < K ? halo_hi[(base + off) * CIN + hc] : (_Float16)0.f;
            B[1][q] = k < K ? halo_lo[(base + off) * CIN + hc] : (_Float16)0.f;
          }
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          acc[mb][nb] = mfma16x16x32h(As[nb][0], B[0], acc[mb][nb]);
          acc[mb][nb] = mfma16x16x32h(As[nb][0], B[1], acc[mb][nb]);
          acc[mb][nb] = mfma16x16x32h(As[nb][1], B[0], acc[mb][nb]);
        }
      }
    }

    // D[n][v]: lane holds channels 16 nb + 4 slot + r (r = 0..3) of voxel 16 mb + row
    bool valid[MB];
    int64_t vox[MB];  // output voxel index within the batch
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int v = wave * 64 + mb * 16 + row;
      const int gz = z0 + v / (TX * TY), gy = y0 + (v / TX) % TY, gx = x0 + v % TX;
      valid[mb] = gz < D && gy < H && gx < W;
      vox[mb] = item + ((int64_t)gz * H + gy) * W + gx;
    }
    // a voxel's channel blocks one after the other, so its row is written by consecutive
    // stores
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int n0 = nb * 16 + slot * 4;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          acc[mb][nb][r] = (acc[mb][nb][r] * inv_x) * inv_w + bn[nb][r];
        }
        if (valid[mb] && n0 < cout) *reinterpret_cast<f4*>(y + vox[mb] * cout + n0) = acc[mb][nb];
      }
    }
    if (stats) {
      // partials over the tile's voxels in one pass: per lane, sums of d = x - s and d^2
      // over its 4 row blocks, with s the value of the wave's first voxel (row 0 of block
      // 0) in that channel; across the 16 lanes of a slot by row rotations; then per wave
      // (count, mean, M2), merged across the 4 waves by Chan's formula
      float cnt = 0.f;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) cnt += valid[mb] ? 1.f : 0.f;
      cnt = row_sum16(cnt);
      const float inv_cnt = cnt > 0.f ? 1.f / cnt : 0.f;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float shift = __shfl(acc[0][nb][r], lane & 48);
          float s1 = 0.f, s2 = 0.f;
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
            const float d = valid[mb] ? acc[mb][nb][r] - shift : 0.f;
            s1 += d;
            s2 = fmaf(d, d, s2);
          }
          s1 = row_sum16(s1);
          s2 = row_sum16(s2);
          if (row == 0) {
            const int n = nb * 16 + slot * 4 + r;
            const float m = s1 * inv_cnt;
            red[wave][n] = shift + m;
            red2[wave][n] = fmaxf(s2 - s1 * m, 0.f);
          }
        }
      if (lane == 0) wcnt[wave] = cnt;
      lds_barrier();
      if (wave == 0) {
        // merge weights of waves 1..3 (the same for every channel), then a lane a channel
        float fw[4], gw[4], na = wcnt[0];
#pragma unroll
        for (int q = 1; q < 4; ++q) {
          const float nq = wcnt[q], nab = na + nq;
          fw[q] = nq > 0.f ? nq / nab : 0.f;
          gw[q] = nq > 0.f ? na * nq / nab : 0.f;
          na = nab;
        }
        for (int n = lane; n < NB * 16; n += 64) {
          float mean = red[0][n], m2 = red2[0][n];
#pragma unroll
          for (int q = 1; q < 4; ++q) {
            const float delta = red[q][n] - mean;
            mean = fmaf(delta, fw[q], mean);
            m2 += red2[q][n] + delta * delta * gw[q];
          }
          if (n < cout)
            stats[((int64_t)blockIdx.y * ntiles + tile) * cout + n] = make_float4(mean, m2, na, 0.f);
        }
      }
    }
    if (tile + 1 < t_end) wave_max(buf ^ 1);
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
__global__ __launch_bounds__(64 * WM* WN, 2) void pw_gemm_kernel(PwArgs a) {
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
  // The next chunk's A (rows of the input) and B (packed weights, whole column groups, no
  // guard) fragments are requested before the current chunk's MFMAs.
  const f2* wl = a.w + nbk0 * 64 + lane;
  const int chunk_stride = a.nblk * 64;
  f2 av[MB], bv[NB];
  {
    const bool ok = 2 * slot < a.cin;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      av[mb] = ok ? *reinterpret_cast<const f2*>(arow[mb]) : f2{0.f, 0.f};
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) bv[nb] = wl[nb * 64];
  }
  for (int chunk = 0; chunk < a.chunks; ++chunk) {
    const int nchunk = chunk + 1 < a.chunks ? chunk + 1 : chunk;
    const bool ok = nchunk * kChunk + 2 * slot < a.cin;
    f2 an[MB], bn[NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      an[mb] = ok ? *reinterpret_cast<const f2*>(arow[mb] + nchunk * kChunk) : f2{0.f, 0.f};
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) bn[nb] = wl[(int64_t)nchunk * chunk_stride + nb * 64];
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          acc[mb][nb] = mfma16x16x4(av[mb][e], bv[nb][e], acc[mb][nb]);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) av[mb] = an[mb];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) bv[nb] = bn[nb];
  }
  // Output voxel of (row m, column n) = base(m) + delta(n), with base(m) the voxel
  // (b, z*KD, y*KH, x*KW) of the output grid and delta(n) the kernel offset (az, ay, ax).
  // Columns are decoded once; each lane's 4 consecutive rows of a block are decoded once
  // and stepped, all in 32-bit arithmetic.
  const int ncols = a.kd * a.kh * a.kw * a.cout;
  const int od = a.id * a.kd, oh = a.ih * a.kh, ow = a.iw * a.kw;
  int col_o[NB], col_delta[NB];
  bool col_ok[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int n = (nbk0 + nb) * 16 + row;
    col_ok[nb] = n < ncols;
    const int o = n % a.cout;
    const int off = n / a.cout;
    const int ax = off % a.kw;
    const int ay = (off / a.kw) % a.kh;
    const int az = off / (a.kw * a.kh);
    col_o[nb] = o;
    col_delta[nb] = (az * oh + ay) * ow + ax;
  }
  const float* bias = a.bias;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int64_t mfirst = m0 + mb * 16 + 4 * slot;
    if (mfirst >= a.M) continue;
    int m32 = (int)mfirst;  // rows fit in 32 bits (checked on the host)
    int xx = m32 % a.iw;
    int t = m32 / a.iw;
    int yy = t % a.ih;
    t /= a.ih;
    int zz = t % a.id;
    int bb = t / a.id;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (mfirst + r < a.M) {
        const int64_t base = (((int64_t)bb * od + zz * a.kd) * oh + yy * a.kh) * (int64_t)ow + xx * a.kw;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          if (!col_ok[nb]) continue;
          float val = acc[mb][nb][r];
          if (bias) val = val + bias[col_o[nb]];
          a.y[(base + col_delta[nb]) * a.cout + col_o[nb]] = val;
        }
      }
      if (++xx == a.iw) {
        xx = 0;
        if (++yy == a.ih) {
          yy = 0;
          if (++zz == a.id) {
            zz = 0;
            ++bb;
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// Split-fp16 transposed convolution (stride == kernel): the pointwise GEMM above on
// v_mfma_f32_16x16x32_f16 with hi*hi + hi*lo + lo*hi products.  A workgroup computes 64
// input voxels x 128 columns (4 waves x 64 x 32).  Per 64-channel block the rows are read
// as contiguous float4 lines, split into fp16 planes in LDS ([row][channel], row stride
// 72 halves); B fragments come from the packed weights (L2 resident).  The epilogue
// stages the tile in LDS and writes each output voxel's channels as contiguous runs; the
// output address is a per-row base (input voxel -> output voxel of offset 0) plus a
// per-column offset (kernel offset and channel), both precomputed in LDS.
// ---------------------------------------------------------------------------------
struct TcArgs {
  const float* x;
  int cin;
  int64_t M;
  const uint4* w16;  // [k-step of 32 channels][16-column block][hi|lo][64 lanes] x 8 fp16
  int nblk, ksteps;
  const float* bias;
  float* y;
  int cout, ncols;
  int kd, kh, kw;
  int id, ih, iw;
  int ntn, nwg;
  int tpb;  // row tiles per workgroup
  float out_scale;
  // pending InstanceNorm (+ LeakyReLU) of the input: (mean, scale, beta, 0) per (b, c), for
  // batch item b = row / vox, vox a multiple of kTcRows (null: the input is final)
  const float4* nrm;
  int act;
  float slope;
  int64_t vox;
};

// The pending normalisation of input channels c..c+3 of batch item b (zero parameters for
// channels past C_in, whose zero loads then stay zero).
__device__ __forceinline__ NormLine tc_norm_line(const TcArgs& a, int64_t b, int c) {
  NormLine nl;
  nl.on = true;
  nl.act = a.act != 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (c + q < a.cin) v = a.nrm[b * a.cin + c + q];
    nl.m[q] = v.x;
    nl.s[q] = v.y;
    nl.b[q] = v.z;
  }
  return nl;
}

// A-plane rows of 80 halves (10 x 16 bytes): the 16-byte fragment reads of a 32-lane half
// (rows r = 0..15, slots s and s + 1) hit (10 r + s) mod 32, all distinct.  Staged output
// rows of 132 floats keep every 4-column run 16-byte aligned for one 16-byte read.
constexpr int kTcRows = 64, kTcCols = 128, kTcKBlock = 64, kTcRowHalves = kTcKBlock + 16;
constexpr int kTcTileStride = kTcCols + 4;  // floats per staged output row

// KREG > 0: the workgroup's weight fragments (at most KREG k-steps of 32 channels) are
// loaded into registers once and serve all its row tiles; KREG = 0: read per k-step.
template <int AR, int KREG>
__global__ __launch_bounds__(256, 2) void tconv_x3_kernel(TcArgs a) {
  constexpr int MB = 4, NB = 2;
  extern __shared__ __align__(16) float lds[];
  _Float16* hi = reinterpret_cast<_Float16*>(lds);
  _Float16* lo = hi + kTcRows * kTcRowHalves;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row = lane & 15;
  const int slot = lane >> 4;
  const int logical = xcd_remap(blockIdx.x, a.nwg);
  const int nt = logical % a.ntn;
  const int blk0 = nt * (kTcCols / 16) + wave * NB;  // first 16-column block of this wave
  auto load_b = [&](h8 (&B)[NB][2], int kstep) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const uint4* w = a.w16 + (((int64_t)kstep * a.nblk + blk0 + nb) * 2) * 64 + lane;
      const uint4 wh = w[0];
      B[nb][0] = *reinterpret_cast<const h8*>(&wh);
      if constexpr (AR == kSplit3) {
        const uint4 wl = w[64];
        B[nb][1] = *reinterpret_cast<const h8*>(&wl);
      }
    }
  };
  h8 BR[KREG > 0 ? KREG : 1][NB][2];
  if constexpr (KREG > 0) {
#pragma unroll
    for (int ks = 0; ks < KREG; ++ks)
      if (ks < a.ksteps) load_b(BR[ks], ks);
  }

  // rows m0.., channels kb..kb+63: 16 float4 lines per row, 4 per thread
  constexpr int kLines = kTcRows * (kTcKBlock / 4) / 256;
  auto load_lines = [&](int64_t m0, int kb, f4 (&lines)[kLines]) {
#pragma unroll
    for (int j = 0; j < kLines; ++j) {
      const int i = tid + 256 * j;
      const int r = i >> 4, c4 = (i & 15) * 4;
      const int64_t m = m0 + r;
      const int c = kb + c4;
      f4 v = {0.f, 0.f, 0.f, 0.f};
      if (m < a.M) {
        const float* src = a.x + m * a.cin + c;
        if (c + 3 < a.cin) {
          v = *reinterpret_cast<const f4*>(src);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (c + q < a.cin) v[q] = src[q];
        }
      }
      lines[j] = v;
    }
  };

  // row tiles tpb * (logical / ntn) .. of column tile nt, one after the other.  KREG > 0
  // (C_in <= 64: one channel block): the next row tile's lines are requested once this
  // tile's are in LDS, so they land during this tile's products and stores
  const int64_t t_begin = (int64_t)(logical / a.ntn) * a.tpb;
  const int64_t t_end = t_begin + a.tpb;
  f4 pre[kLines];
  if constexpr (KREG > 0) {
    if (t_begin * kTcRows < a.M) load_lines(t_begin * kTcRows, 0, pre);
  }
  for (int64_t t = t_begin; t < t_end; ++t) {
    const int64_t m0 = t * kTcRows;
    if (m0 >= a.M) break;
    f4 acc[MB][NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f4{0.f, 0.f, 0.f, 0.f};

    for (int kb = 0; kb < a.cin; kb += kTcKBlock) {
      // all lines requested before the barrier
      f4 lines[kLines];
      if constexpr (KREG > 0) {
#pragma unroll
        for (int j = 0; j < kLines; ++j) lines[j] = pre[j];
      } else {
        load_lines(m0, kb, lines);
      }
      // the pending normalisation of this thread's channel quad (the same for all its
      // lines; a row tile lies in one batch item, vox being a multiple of the tile rows)
      NormLine nl{};
      if (a.nrm) nl = tc_norm_line(a, m0 / a.vox, kb + (tid & 15) * 4);
      __syncthreads();  // the previous block's fragments have been read
#pragma unroll
      for (int j = 0; j < kLines; ++j) {
        const int i = tid + 256 * j;
        const int r = i >> 4, c4 = (i & 15) * 4;
        f4 v = lines[j];
        if (a.nrm && m0 + r < a.M) v = norm_apply4(v, nl, a.slope);
        h4 hv, lv;
        to_operand4<AR>(v, hv, lv);
        *reinterpret_cast<h4*>(hi + r * kTcRowHalves + c4) = hv;
        if constexpr (AR == kSplit3) *reinterpret_cast<h4*>(lo + r * kTcRowHalves + c4) = lv;
      }
      __syncthreads();
      if constexpr (KREG > 0) {
        if (t + 1 < t_end && m0 + kTcRows < a.M) load_lines(m0 + kTcRows, 0, pre);
      }
#pragma unroll
      for (int ks = 0; ks < kTcKBlock / 32; ++ks) {
        const int kstep = kb / 32 + ks;
        if (kstep >= a.ksteps) break;
        h8 A[MB][2];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const int off = (mb * 16 + row) * kTcRowHalves + ks * 32 + slot * 8;
          A[mb][0] = *reinterpret_cast<const h8*>(hi + off);
          if constexpr (AR == kSplit3) A[mb][1] = *reinterpret_cast<const h8*>(lo + off);
        }
        if constexpr (KREG > 0) {
          // k-steps kb / 32 + ks < ksteps <= KREG
          mma_products<AR>(acc, A, BR[kb / 32 + ks < KREG ? kb / 32 + ks : 0]);
        } else {
          h8 B[NB][2];
          load_b(B, kstep);
          mma_products<AR>(acc, A, B);
        }
      }
    }

    // epilogue: tile T[r][c] (scaled, + bias) in LDS, then runs of contiguous channels
    float* tile = lds;
    int64_t* row_base = reinterpret_cast<int64_t*>(lds + kTcRows * kTcTileStride);
    int* col_off = reinterpret_cast<int*>(row_base + kTcRows);
    const int od = a.id * a.kd, oh = a.ih * a.kh, ow = a.iw * a.kw;
    __syncthreads();  // the A planes are no longer read
    if (tid < kTcRows) {
      const int64_t m = m0 + tid;
      int64_t base = -1;
      if (m < a.M) {
        const int xx = (int)(m % a.iw);
        int64_t t = m / a.iw;
        const int yy = (int)(t % a.ih);
        t /= a.ih;
        const int zz = (int)(t % a.id);
        const int64_t bb = t / a.id;
        base = ((bb * od + (int64_t)zz * a.kd) * oh + (int64_t)yy * a.kh) * ow + (int64_t)xx * a.kw;
      }
      row_base[tid] = base;
    } else if (tid < kTcRows + kTcCols) {
      const int cl = tid - kTcRows;
      const int n = nt * kTcCols + cl;
      int off = -1;
      if (n < a.ncols) {
        const int j = n / a.cout, o = n - j * a.cout;
        const int ax = j % a.kw, ay = (j / a.kw) % a.kh, az = j / (a.kw * a.kh);
        off = ((az * oh + ay) * ow + ax) * a.cout + o;
      }
      col_off[cl] = off;
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int cl = (wave * NB + nb) * 16 + row;
      const int n = nt * kTcCols + cl;
      const float bias_n = (a.bias && n < a.ncols) ? a.bias[n % a.cout] : 0.f;
      const bool has_bias = a.bias != nullptr;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = acc[mb][nb][r] * a.out_scale;
          tile[(mb * 16 + 4 * slot + r) * kTcTileStride + cl] = has_bias ? v + bias_n : v;
        }
    }
    __syncthreads();
    if (a.cout % 4 == 0) {
      // 4 consecutive columns are 4 consecutive channels of one output voxel: 16-byte stores
      for (int e4 = tid; e4 < kTcRows * kTcCols / 4; e4 += 256) {
        const int r = e4 >> 5, cl = (e4 & 31) * 4;
        const int64_t base = row_base[r];
        const int off = col_off[cl];
        if (base >= 0 && off >= 0) {
          *reinterpret_cast<f4*>(a.y + base * a.cout + off) =
              *reinterpret_cast<const f4*>(tile + r * kTcTileStride + cl);
        }
      }
    } else {
      for (int e = tid; e < kTcRows * kTcCols; e += 256) {
        const int r = e >> 7, cl = e & (kTcCols - 1);
        const int64_t base = row_base[r];
        const int off = col_off[cl];
        if (base >= 0 && off >= 0) a.y[base * a.cout + off] = tile[r * kTcTileStride + cl];
      }
    }
  }  // row tiles
}

// Packing: words ((kstep * nblk + nb) * 2 + part) * 64 + lane = part 0: hi, part 1: lo h8 of
// scale * W[k][n], k = 32 * kstep + 8 * (lane / 16) + q, n = 16 * nb + lane % 16, where
// column n = ((az * KH + ay) * KW + ax) * C_out + o reads the reference weight
// (C_out, kD, kH, kW, C_in) at (o, az, ay, ax, k).
__global__ void pack_tconv_weight_x3_kernel(const float* __restrict__ w, uint4* __restrict__ out,
                                            int cout, int koff, int cin, int ksteps, int nblk,
                                            float scale, int arith) {
  const int64_t total = (int64_t)ksteps * nblk * 64;
  const int ncols = koff * cout;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(i % 64);
    const int64_t r = i / 64;
    const int nb = (int)(r % nblk);
    const int kstep = (int)(r / nblk);
    const int n = nb * 16 + (lane & 15);
    h8 hv, lv;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int k = kstep * 32 + 8 * (lane >> 4) + q;
      float v = 0.f;
      if (n < ncols && k < cin) {
        const int o = n % cout, off = n / cout;
        v = w[((int64_t)o * koff + off) * cin + k] * scale;
      }
      _Float16 hh, ll;
      if (arith == kBf16)
        to_operand<kBf16>(v, hh, ll);
      else
        to_operand<kSplit3>(v, hh, ll);
      hv[q] = hh;
      lv[q] = ll;
    }
    const int64_t word = (i - lane) * 2 + lane;
    out[word] = *reinterpret_cast<const uint4*>(&hv);
    out[word + 64] = *reinterpret_cast<const uint4*>(&lv);
  }
}

// ---------------------------------------------------------------------------------
// 1x1x1 convolution with few outputs (segmentation head): one thread per voxel, the
// weights in LDS; s = fma chain over input channels, then + bias.
// ---------------------------------------------------------------------------------
// Pending InstanceNorm (+ LeakyReLU) of one input element (the apply pass's operations).
__device__ __forceinline__ float norm_apply1(float v, float4 p, int act, float slope) {
  float t = fmaf(v - p.x, p.y, p.z);
  return act ? fmaxf(slope * t, t) : t;
}

__global__ __launch_bounds__(256) void conv1x1_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ w,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ y, int64_t nvox,
                                                      int cin, int cout,
                                                      const float4* __restrict__ nrm, int act,
                                                      float slope, int64_t item_vox) {
  extern __shared__ float ws[];  // cout * cin
  for (int i = threadIdx.x; i < cout * cin; i += blockDim.x) ws[i] = w[i];
  __syncthreads();
  const int64_t vox = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (vox >= nvox) return;
  const float* xr = x + vox * cin;
  const float4* pr = nrm ? nrm + (vox / item_vox) * cin : nullptr;
  for (int o = 0; o < cout; ++o) {
    float s = 0.f;
    const float* wr = ws + o * cin;
    for (int c = 0; c < cin; ++c) {
      const float xv = pr ? norm_apply1(xr[c], pr[c], act, slope) : xr[c];
      s = fmaf(xv, wr[c], s);
    }
    y[vox * cout + o] = bias ? s + bias[o] : s;
  }
}

// Head for narrow inputs (C_in <= 64, a multiple of 4): the block's 256 input rows are
// loaded into LDS with coalesced float4 reads (rows padded to C_in + 4 floats, so a row is
// read back as float4s without bank conflicts), each thread keeps its voxel's row in
// registers and forms its outputs (fma chain over channels, then + bias) with the weights
// from scalar loads (uniform addresses in the constant address space), and the outputs
// leave as one run.
template <int CIN>
__global__ __launch_bounds__(256) void conv1x1_staged_kernel(const float* __restrict__ x,
                                                             const float* __restrict__ w,
                                                             const float* __restrict__ bias,
                                                             float* __restrict__ y, int64_t nvox,
                                                             int cout,
                                                             const float4* __restrict__ nrm,
                                                             int act, float slope,
                                                             int64_t item_vox) {
  typedef const __attribute__((address_space(4))) float* cfloat_p;
  constexpr int cin = CIN, cin4 = CIN / 4, xstride = CIN + 4;
  extern __shared__ __align__(16) float smem[];
  float* xs = smem;                   // 256 * (cin + 4)
  float* os = xs + 256 * xstride;     // 256 * cout
  const cfloat_p wc = (cfloat_p)w;
  const cfloat_p bc = (cfloat_p)bias;
  const int64_t v0 = blockIdx.x * (int64_t)blockDim.x;
  const int nv = (int)(nvox - v0 < 256 ? nvox - v0 : 256);
  const f4* src = reinterpret_cast<const f4*>(x + v0 * cin);
  const int total4 = nv * cin4;
  // a full block holds 256 * cin4 float4s: cin4 per thread, all loads issued before use
  f4 v[cin4];
#pragma unroll
  for (int j = 0; j < cin4; ++j) {
    const int e4 = j * 256 + (int)threadIdx.x;
    v[j] = e4 < total4 ? src[e4] : f4{0.f, 0.f, 0.f, 0.f};
  }
  if (nrm) {
    // batch item of the block's first voxel; rows from `split` on belong to the next item
    const int64_t item0 = v0 / item_vox;
    const int64_t split = (item0 + 1) * item_vox - v0;
    auto apply = [&](f4& val, const float4* pr) {
      val[0] = norm_apply1(val[0], pr[0], act, slope);
      val[1] = norm_apply1(val[1], pr[1], act, slope);
      val[2] = norm_apply1(val[2], pr[2], act, slope);
      val[3] = norm_apply1(val[3], pr[3], act, slope);
    };
    if constexpr (256 % cin4 == 0) {
      // every element of this thread lies in channel group tid % cin4
      const int c = ((int)threadIdx.x % cin4) * 4;
      float4 pa[4], pb[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) pa[q] = nrm[item0 * cin + c + q];
#pragma unroll
      for (int q = 0; q < 4; ++q) pb[q] = split < nv ? nrm[(item0 + 1) * cin + c + q] : pa[q];
#pragma unroll
      for (int j = 0; j < cin4; ++j) {
        const int r = (j * 256 + (int)threadIdx.x) / cin4;
        apply(v[j], r >= split ? pb : pa);
      }
    } else {
#pragma unroll
      for (int j = 0; j < cin4; ++j) {
        const int e4 = j * 256 + (int)threadIdx.x;
        const int r = e4 / cin4;
        if (e4 < total4)
          apply(v[j], nrm + (item0 + (r >= split ? 1 : 0)) * cin + (e4 - r * cin4) * 4);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < cin4; ++j) {
    const int e4 = j * 256 + (int)threadIdx.x;
    const int r = e4 / cin4;
    if (e4 < total4) *reinterpret_cast<f4*>(xs + r * xstride + (e4 - r * cin4) * 4) = v[j];
  }
  __syncthreads();
  if ((int)threadIdx.x < nv) {
    f4 xr[cin4];
#pragma unroll
    for (int c4 = 0; c4 < cin4; ++c4)
      xr[c4] = *reinterpret_cast<const f4*>(xs + threadIdx.x * xstride + c4 * 4);
    for (int o = 0; o < cout; ++o) {
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < cin; ++c) s = fmaf(xr[c >> 2][c & 3], wc[o * cin + c], s);
      os[threadIdx.x * cout + o] = bias ? s + bc[o] : s;
    }
  }
  __syncthreads();
  float* dst = y + v0 * cout;
  for (int e = threadIdx.x; e < nv * cout; e += blockDim.x) dst[e] = os[e];
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
  // the kernels hold a voxel's offset inside its batch item in 32 bits (the output has no
  // more voxels than the input)
  require((int64_t)in_size[0] * in_size[1] * in_size[2] < (1LL << 31),
          "convolution input exceeds 2^31 voxels per batch item");
  return g;
}

// Column blocks of the packed conv weights are padded to whole groups of kBlockGroup so
// that every variant's workgroup (WN*NB <= 8 blocks) reads its weights unguarded.
constexpr int kBlockGroup = 8;

int conv_packed_nblk(int cout) { return (int)(ceil_div(ceil_div(cout, 16), kBlockGroup) * kBlockGroup); }

int64_t conv_packed_floats(int cout, const int* ksize, int c1, int c2) {
  const int64_t taps = (int64_t)ksize[0] * ksize[1] * ksize[2];
  const int64_t chunks = ceil_div(c1, kChunk) + ceil_div(c2, kChunk);
  const int64_t nblk = conv_packed_nblk(cout);
  return chunks * taps * nblk * 64 * 2;
}

void conv_pack_weight(const float* d_w, int cout, const int* ksize, int c1, int c2,
                      float* d_packed, hipStream_t st) {
  require(cout >= 1 && c1 >= 1 && c2 >= 0, "invalid convolution channel counts");
  const int taps = ksize[0] * ksize[1] * ksize[2];
  const int chunks1 = (int)ceil_div(c1, kChunk);
  const int chunks = chunks1 + (int)ceil_div(c2, kChunk);
  const int nblk = conv_packed_nblk(cout);
  const int64_t total = (int64_t)chunks * taps * nblk * 64;
  const int blocks = (int)std::min<int64_t>(ceil_div(total, 256), 65536);
  hipLaunchKernelGGL(pack_conv_weight_kernel, dim3(blocks), dim3(256), 0, st, d_w,
                     reinterpret_cast<f2*>(d_packed), cout, taps, c1, c2, chunks1, chunks, nblk);
  launch_check("conv3d_pack_weight");
}

namespace {

struct IgemmPlan {
  Variant v;
  Box box;
  bool async;
};

IgemmPlan plan_igemm(const ConvGeom& g, int cout, int c1, int c2) {
  const bool stride1 = g.s[0] == 1 && g.s[1] == 1 && g.s[2] == 1;
  const int64_t vox = (int64_t)g.out[0] * g.out[1] * g.out[2];
  IgemmPlan p{};
  if (cout <= 32)
    p.v = stride1 ? kVarA : kVarD;
  else if (cout <= 64)
    p.v = stride1 ? kVarB : kVarD;
  else
    p.v = (vox * g.batch <= 8192) ? kVarE : kVarC;
  // The asynchronous path needs whole 8-channel lines and a double-buffered halo that fits.
  // The register-staged halo measured faster than the DMA path on every liver layer
  // (70-82 % vs 63-78 % of fp32 MFMA peak), so the DMA path is opt-in.
  static const char* halo_mode = std::getenv("NNX_IGEMM_HALO");
  p.async = halo_mode && std::string(halo_mode) == "async" && c1 % kChunk == 0 &&
            c2 % kChunk == 0;
  bool found = false;
  if (p.async) {
    try {
      p.box = choose_box(p.v, g, true);
      found = true;
    } catch (const Error&) {
      p.async = false;
    }
  }
  if (!found) p.box = choose_box(p.v, g, false);
  return p;
}

}  // namespace

int conv_stats_tiles(const ConvGeom& g, int cout, int c1, int c2) {
  const Box box = plan_igemm(g, cout, c1, c2).box;
  return (int)(ceil_div(g.out[0], box.z) * ceil_div(g.out[1], box.y) * ceil_div(g.out[2], box.x));
}

namespace {

// Geometry, box and grid fields shared by both implicit-GEMM kernels.
IgemmArgs igemm_args(const float* x1, int c1, const float* x2, int c2, const float* bias,
                     float* y, const ConvGeom& g, int cout, const Variant& v, const Box& box,
                     float4* stats, const PendingNorm& n1, const PendingNorm& n2) {
  require(!(n1.params && n2.params) || n1.slope == n2.slope,
          "pending normalisations of one convolution must share the LeakyReLU slope");
  IgemmArgs a{};
  a.nrm0 = n1.params;
  a.nrm1 = n2.params;
  a.act0 = n1.act ? 1 : 0;
  a.act1 = n2.act ? 1 : 0;
  a.slope = n1.params ? n1.slope : n2.slope;
  a.x0 = x1;
  a.x1 = x2;
  a.c0 = c1;
  a.c1 = c2;
  a.chunks0 = (int)ceil_div(c1, kChunk);
  a.chunks = a.chunks0 + (int)ceil_div(c2, kChunk);
  a.bias = bias;
  a.y = y;
  a.id = g.in[0];
  a.ih = g.in[1];
  a.iw = g.in[2];
  a.od = g.out[0];
  a.oh = g.out[1];
  a.ow = g.out[2];
  a.cout = cout;
  a.nblk = conv_packed_nblk(cout);
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
  require((box.x & (box.x - 1)) == 0 && (box.y & (box.y - 1)) == 0, "box dims must be powers of two");
  a.lbx = __builtin_ctz(box.x);
  a.lbxy = __builtin_ctz(box.x * box.y);
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
  a.stats = stats;
  a.out_scale = 1.0f;
  return a;
}

// Algorithmic work: 2*C_in*C_out*taps per output voxel; bytes: input, output, weights once.
void igemm_work(const ConvGeom& g, int c1, int c2, int cout, double* flops, double* bytes) {
  const double out_vox = (double)g.batch * g.out[0] * g.out[1] * g.out[2];
  const double in_vox = (double)g.batch * g.in[0] * g.in[1] * g.in[2];
  const double taps = (double)g.k[0] * g.k[1] * g.k[2];
  *flops = 2.0 * (c1 + c2) * cout * taps * out_vox;
  *bytes = 4.0 * (in_vox * (c1 + c2) + out_vox * cout + taps * (c1 + c2) * cout);
}

}  // namespace

void conv3d_igemm(const float* x1, int c1, const float* x2, int c2, const float* packed,
                  const float* bias, float* y, const ConvGeom& g, int cout, hipStream_t st,
                  float4* stats, const PendingNorm& n1, const PendingNorm& n2) {
  require(x1 && y && packed, "convolution pointers must not be null");
  require(c1 >= 1 && (c2 == 0 || x2), "invalid convolution inputs");
  const IgemmPlan plan = plan_igemm(g, cout, c1, c2);
  const Variant v = plan.v;
  // the DMA halo path copies lines unchanged: pending normalisations need the register path
  const bool async = plan.async && !n1.params && !n2.params;
  IgemmArgs a = igemm_args(x1, c1, x2, c2, bias, y, g, cout, v, plan.box, stats, n1, n2);
  a.w = reinterpret_cast<const f2*>(packed);
  double flops, bytes;
  igemm_work(g, c1, c2, cout, &flops, &bytes);
  if (v.MB == 8)
    launch_igemm<8, 2, 4, 1>(a, a.nwg, async, st, flops, bytes);
  else if (v.MB == 4 && v.WN == 1)
    launch_igemm<4, 4, 4, 1>(a, a.nwg, async, st, flops, bytes);
  else if (v.MB == 4)
    launch_igemm<4, 4, 2, 2>(a, a.nwg, async, st, flops, bytes);
  else if (v.WN == 1)
    launch_igemm<2, 4, 4, 1>(a, a.nwg, async, st, flops, bytes);
  else
    launch_igemm<2, 4, 2, 2>(a, a.nwg, async, st, flops, bytes);
}

// ---- split-fp16 ("x3") implicit GEMM ----------------------------------------------

float split_weight_scale(double max_abs) {
  require(std::isfinite(max_abs) && max_abs >= 0.0, "weight magnitude must be finite");
  if (max_abs == 0.0) return 1.0f;
  // the power of two that brings max |w| into [2^14, 2^15): high halves stay below the
  // fp16 maximum (65504) and low halves of all but tiny weights stay normal.  Below 2^-113
  // the scale stops at 2^127, the largest float power of two (max |w| then lands lower).
  int e;
  std::frexp(max_abs, &e);  // max_abs = m * 2^e, m in [0.5, 1)
  return std::ldexp(1.0f, std::min(15 - e, 127));
}

int conv_x3_groups(const int* ksize) { return (ksize[0] * ksize[1] * ksize[2] + 3) / 4; }
int64_t conv_x3_packed_bytes(int cout, const int* ksize, int c1, int c2) {
  const int64_t chunks = ceil_div(c1, kChunk) + ceil_div(c2, kChunk);
  return chunks * conv_x3_groups(ksize) * conv_packed_nblk(cout) * 64 * 32;
}

void conv_x3_pack_weight(const float* d_w, int cout, const int* ksize, int c1, int c2,
                         float scale, void* d_packed, hipStream_t st, int arith) {
  require(cout >= 1 && c1 >= 1 && c2 >= 0, "invalid convolution channel counts");
  require(arith == kSplit3 || arith == kBf16, "unknown convolution arithmetic");
  require(scale > 0.f && std::isfinite(scale), "weight scale must be positive");
  const int taps = ksize[0] * ksize[1] * ksize[2];
  const int chunks1 = (int)ceil_div(c1, kChunk);
  const int chunks = chunks1 + (int)ceil_div(c2, kChunk);
  const int groups = conv_x3_groups(ksize);
  const int nblk = conv_packed_nblk(cout);
  const int64_t total = (int64_t)chunks * groups * nblk * 64;
  const int blocks = (int)std::min<int64_t>(ceil_div(total, 256), 65536);
  hipLaunchKernelGGL(pack_conv_weight_x3_kernel, dim3(blocks), dim3(256), 0, st, d_w,
                     reinterpret_cast<uint4*>(d_packed), cout, taps, c1, c2, chunks1, chunks,
                     groups, nblk, scale, arith);
  launch_check("conv3d_x3_pack_weight");
}

namespace {

// register-staged kernels (strided convolutions, whose halos exceed the staged budget)
constexpr Variant kX3C{2, 4, 2, 2};  // M 64,  N 128
constexpr Variant kX3F{2, 2, 2, 2};  // M 64,  N 64
// halo voxels one workgroup can stage in registers (2 lines per voxel)
constexpr int64_t kX3MaxHalo = (int64_t)kX3MaxLines * kX3Threads / 2;

// LDS per workgroup of the weight-staged kernel that keeps 3 workgroups on a CU
constexpr int64_t kX3sLdsBytes = 53 * 1024;
constexpr Variant kX3S{4, 2, 4, 1};  // weight-staged: M 256, N 32

struct X3Plan {
  Variant v;
  Box box;
  bool staged;  // igemm_x3s_kernel
};

bool x3_groups_supported(int ntg) { return ntg == 1 || ntg == 3 || ntg == 7; }

// Stride-1 convolutions use the weight-staged kernel (M 256, N 32 per workgroup) when a box
// fits its LDS budget; the others (strided) use the register-staged kernel.
X3Plan plan_x3(const ConvGeom& g, int cout) {
  require(x3_groups_supported(conv_x3_groups(g.k)),
          "split convolution supports 1-4, 9-12 or 25-28 kernel taps");
  X3Plan p{};
  const int ntg = conv_x3_groups(g.k);
  const int64_t wbytes = (int64_t)x3s_lds_bytes(0, ntg, kX3S.NB * kX3S.WN);
  try {
    p.box = choose_box(kX3S, g, false, (kX3sLdsBytes - wbytes) / 32);
    p.v = kX3S;
    p.staged = true;
    return p;
  } catch (const Error&) {
  }
  // N 64 up to 64 output channels, and wherever N 128 would leave fewer than 4 workgroups
  // a CU; N 128 (half the halo staging per output channel) otherwise
  p.v = kX3F;
  p.box = choose_box(kX3F, g, false, kX3MaxHalo);
  if (cout > 64) {
    const Box wide = choose_box(kX3C, g, false, kX3MaxHalo);
    if (g.batch * wide.tiles * ceil_div(cout, kX3C.n()) >= 1024) {
      p.v = kX3C;
      p.box = wide;
    }
  }
  p.staged = false;
  return p;
}

}  // namespace

bool conv_x3_supported(const int* ksize, const int* stride, int cout) {
  // the halo box depends on kernel and stride only; probe with a large volume
  const int big[3] = {256, 256, 256};
  try {
    plan_x3(make_conv_geom(1, big, ksize, stride), cout);
    return true;
  } catch (const Error&) {
    return false;
  }
}

int conv_x3_stats_tiles(const ConvGeom& g, int cout) {
  const Box box = plan_x3(g, cout).box;
  return (int)(ceil_div(g.out[0], box.z) * ceil_div(g.out[1], box.y) * ceil_div(g.out[2], box.x));
}

void conv3d_x3(const float* x1, int c1, const float* x2, int c2, const void* packed,
               float scale, const float* bias, float* y, const ConvGeom& g, int cout,
               hipStream_t st, float4* stats, const PendingNorm& n1, const PendingNorm& n2,
               int arith) {
  require(x1 && y && packed, "convolution pointers must not be null");
  require(c1 >= 1 && (c2 == 0 || x2), "invalid convolution inputs");
  require(scale > 0.f && std::isfinite(scale), "weight scale must be positive");
  require(arith == kSplit3 || arith == kBf16, "unknown convolution arithmetic");
  const X3Plan plan = plan_x3(g, cout);
  const Variant v = plan.v;
  IgemmArgs a = igemm_args(x1, c1, x2, c2, bias, y, g, cout, v, plan.box, stats, n1, n2);
  a.w16 = reinterpret_cast<const uint4*>(packed);
  a.ntg = conv_x3_groups(g.k);
  a.out_scale = 1.0f / scale;
  require(plan.staged || (int64_t)a.hz * a.hy * a.hx <= kX3MaxHalo,
          "split convolution halo exceeds the staging");
  double flops, bytes;
  igemm_work(g, c1, c2, cout, &flops, &bytes);
  const bool vec = c1 % kChunk == 0 && c2 % kChunk == 0;
  if (plan.staged) {
    // whole 32-column blocks and 16-byte aligned rows: the epilogue writes float4 words
    a.vstore = cout % 32 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0;
    launch_x3s<4, 2, 4, 1>(a, vec, arith, st, flops, bytes);
    return;
  }
  if (v.NB == 4)
    launch_x3<2, 4, 2, 2>(a, vec, arith, st, flops, bytes);
  else
    launch_x3<2, 2, 2, 2>(a, vec, arith, st, flops, bytes);
}

int conv_direct_stats_tiles(const int* size, bool split) {
  if (split)
    return (int)(ceil_div(size[0], kDirX3Tz) * ceil_div(size[1], kDirX3Ty) *
                 ceil_div(size[2], kDirX3Tx));
  return (int)(ceil_div(size[0], kDirTz) * ceil_div(size[1], kDirTy) * ceil_div(size[2], kDirTx));
}

void conv3d_direct_cin1(const float* x, const float* w, const float* bias, float* y, int batch,
                        const int* size, int cout, hipStream_t st, float4* stats, float wscale,
                        int cin) {
  require(x && w && y, "convolution pointers must not be null");
  require(cin == 1 || (wscale > 0.f && (cin == 2 || cin == 4)),
          "the direct convolution takes 1 input channel, or 2 or 4 with split products");
  require(cout >= 4 && cout <= 64 && cout % 4 == 0,
          "one-channel direct convolution supports 4..64 outputs in steps of 4");
  require(batch >= 1 && batch <= 65535, "invalid convolution batch");
  require(wscale == 0.f || (wscale > 0.f && std::isfinite(wscale)),
          "weight scale must be positive (split products) or 0 (float32 products)");
  const int64_t S = (int64_t)size[0] * size[1] * size[2];
  require(S >= 1, "empty convolution input");
  const int64_t nvox = (int64_t)batch * S;
  const bool split = wscale > 0.f;
  const int tiles_y = (int)ceil_div(size[1], split ? kDirX3Ty : kDirTy);
  const int tiles_x = (int)ceil_div(size[2], split ? kDirX3Tx : kDirTx);
  const int64_t tiles = conv_direct_stats_tiles(size, split);
  require(tiles < (1LL << 31), "convolution volume too large");
  const dim3 grid((unsigned)tiles, (unsigned)batch);
  const size_t lds = (size_t)256 * (cout + 1) * sizeof(float);
  const double bytes = 4.0 * (double)nvox * (cin + cout);
  if (split) {
    // split products on MFMA: the output write bounds it (reported against HBM).  Each
    // block takes kDirX3TilesPerBlock consecutive tiles (weights split once per block).
    const int tpb = kDirX3TilesPerBlock;
    const dim3 grid_x3((unsigned)ceil_div(tiles, tpb), (unsigned)batch);
    ProfScope prof("conv3d_direct_cin1_x3", 0.0, bytes, st);
    switch (cout / 4) {
#define NNX_DIRECT_X3_CASE(Q)                                                                  \
  case Q:                                                                                      \
    if (cin == 1)                                                                              \
      hipLaunchKernelGGL((direct_cin1_x3_kernel<4 * Q, 1>), grid_x3, dim3(256), 0, st, x, w,    \
                         wscale, bias, y, size[0], size[1], size[2], tiles_y, tiles_x,          \
                         (int)tiles, tpb, stats);                                               \
    else if (cin == 2)                                                                         \
      hipLaunchKernelGGL((direct_cin1_x3_kernel<4 * Q, 2>), grid_x3, dim3(256), 0, st, x, w,    \
                         wscale, bias, y, size[0], size[1], size[2], tiles_y, tiles_x,          \
                         (int)tiles, tpb, stats);                                               \
    else                                                                                       \
      hipLaunchKernelGGL((direct_cin1_x3_kernel<4 * Q, 4>), grid_x3, dim3(256), 0, st, x, w,    \
                         wscale, bias, y, size[0], size[1], size[2], tiles_y, tiles_x,          \
                         (int)tiles, tpb, stats);                                               \
    break;
      NNX_DIRECT_X3_CASE(1) NNX_DIRECT_X3_CASE(2) NNX_DIRECT_X3_CASE(3) NNX_DIRECT_X3_CASE(4)
      NNX_DIRECT_X3_CASE(5) NNX_DIRECT_X3_CASE(6) NNX_DIRECT_X3_CASE(7) NNX_DIRECT_X3_CASE(8)
      NNX_DIRECT_X3_CASE(9) NNX_DIRECT_X3_CASE(10) NNX_DIRECT_X3_CASE(11) NNX_DIRECT_X3_CASE(12)
      NNX_DIRECT_X3_CASE(13) NNX_DIRECT_X3_CASE(14) NNX_DIRECT_X3_CASE(15) NNX_DIRECT_X3_CASE(16)
#undef NNX_DIRECT_X3_CASE
    }
    launch_check("conv3d_direct_small_cin_split");
    return;
  }
  ProfScope prof("conv3d_direct_cin1", 2.0 * 27 * cout * (double)nvox, bytes, st);
  switch (cout / 4) {
#define NNX_DIRECT_CASE(Q)                                                                     \
  case Q:                                                                                      \
    hipLaunchKernelGGL(direct_cin1_kernel<4 * Q>, grid, dim3(256), lds, st, x, w, bias, y,     \
                       size[0], size[1], size[2], tiles_y, tiles_x, stats);                    \
    break;
    NNX_DIRECT_CASE(1) NNX_DIRECT_CASE(2) NNX_DIRECT_CASE(3) NNX_DIRECT_CASE(4)
    NNX_DIRECT_CASE(5) NNX_DIRECT_CASE(6) NNX_DIRECT_CASE(7) NNX_DIRECT_CASE(8)
    NNX_DIRECT_CASE(9) NNX_DIRECT_CASE(10) NNX_DIRECT_CASE(11) NNX_DIRECT_CASE(12)
    NNX_DIRECT_CASE(13) NNX_DIRECT_CASE(14) NNX_DIRECT_CASE(15) NNX_DIRECT_CASE(16)
#undef NNX_DIRECT_CASE
  }
  launch_check("conv3d_direct_small_cin");
}

int tconv_packed_nblk(int64_t ncols) { return (int)(ceil_div(ceil_div(ncols, 16), kBlockGroup) * kBlockGroup); }

int64_t tconv_packed_floats(int cout, const int* ksize, int cin) {
  const int64_t koff = (int64_t)ksize[0] * ksize[1] * ksize[2];
  return ceil_div(cin, kChunk) * tconv_packed_nblk(koff * cout) * 64 * 2;
}

void tconv_pack_weight(const float* d_w, int cout, const int* ksize, int cin, float* d_packed,
                       hipStream_t st) {
  require(cout >= 1 && cin >= 1, "invalid transposed-convolution channel counts");
  const int koff = ksize[0] * ksize[1] * ksize[2];
  const int chunks = (int)ceil_div(cin, kChunk);
  const int nblk = tconv_packed_nblk((int64_t)koff * cout);
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
  a.nblk = tconv_packed_nblk(ncols);
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
  require(a.M < (1LL << 31) - 64, "transposed-convolution input too large");
  a.ntn = (int)ceil_div(ncols, 16 * NB * WN);
  const int64_t nwg = ceil_div(a.M, 16 * MB * WM) * a.ntn;
  require(nwg < (1LL << 31), "transposed-convolution grid too large");
  a.nwg = (int)nwg;
  ProfScope prof("tconv3d_gemm", 2.0 * (double)a.M * cin * ncols,
                 4.0 * ((double)a.M * (cin + ncols) + (double)cin * ncols), st);
  hipLaunchKernelGGL((pw_gemm_kernel<MB, NB, WM, WN>), dim3(a.nwg), dim3(64 * WM * WN), 0, st, a);
  launch_check("tconv3d_gemm");
}

int64_t tconv_x3_packed_bytes(int cout, const int* ksize, int cin) {
  const int64_t koff = (int64_t)ksize[0] * ksize[1] * ksize[2];
  return ceil_div(cin, 32) * tconv_packed_nblk(koff * cout) * 128 * 16;
}

void tconv_x3_pack_weight(const float* d_w, int cout, const int* ksize, int cin, float scale,
                          void* d_packed, hipStream_t st, int arith) {
  require(cout >= 1 && cin >= 1, "invalid transposed-convolution channel counts");
  require(arith == kSplit3 || arith == kBf16, "unknown transposed-convolution arithmetic");
  require(scale > 0.f && std::isfinite(scale), "weight scale must be positive");
  const int koff = ksize[0] * ksize[1] * ksize[2];
  const int ksteps = (int)ceil_div(cin, 32);
  const int nblk = tconv_packed_nblk((int64_t)koff * cout);
  const int64_t total = (int64_t)ksteps * nblk * 64;
  const int blocks = (int)std::min<int64_t>(ceil_div(total, 256), 65536);
  hipLaunchKernelGGL(pack_tconv_weight_x3_kernel, dim3(blocks), dim3(256), 0, st, d_w,
                     reinterpret_cast<uint4*>(d_packed), cout, koff, cin, ksteps, nblk, scale,
                     arith);
  launch_check("tconv3d_split_pack_weight");
}

bool tconv_norm_on_load(const int* in_size) {
  return (int64_t)in_size[0] * in_size[1] * in_size[2] % kTcRows == 0;
}

void tconv3d_x3(const float* x, int cin, const void* packed, float scale, const float* bias,
                float* y, int batch, const int* in_size, int cout, const int* ksize,
                hipStream_t st, int arith, const PendingNorm& norm) {
  require(x && packed && y, "transposed-convolution pointers must not be null");
  require(cin >= 1 && cout >= 1, "invalid transposed-convolution channel counts");
  require(arith == kSplit3 || arith == kBf16, "unknown transposed-convolution arithmetic");
  require(scale > 0.f && std::isfinite(scale), "weight scale must be positive");
  for (int i = 0; i < 3; ++i) require(ksize[i] >= 1 && in_size[i] >= 1, "invalid tconv geometry");
  TcArgs a{};
  a.x = x;
  a.cin = cin;
  a.M = (int64_t)batch * in_size[0] * in_size[1] * in_size[2];
  a.w16 = reinterpret_cast<const uint4*>(packed);
  a.ksteps = (int)ceil_div(cin, 32);
  a.ncols = ksize[0] * ksize[1] * ksize[2] * cout;
  a.nblk = tconv_packed_nblk(a.ncols);
  a.bias = bias;
  a.y = y;
  a.cout = cout;
  a.kd = ksize[0];
  a.kh = ksize[1];
  a.kw = ksize[2];
  a.id = in_size[0];
  a.ih = in_size[1];
  a.iw = in_size[2];
  a.out_scale = 1.0f / scale;
  a.nrm = norm.params;
  a.act = norm.act ? 1 : 0;
  a.slope = norm.slope;
  a.vox = (int64_t)in_size[0] * in_size[1] * in_size[2];
  require(!a.nrm || a.vox % kTcRows == 0,
          "a pending input norm needs whole row tiles per batch item (tconv_norm_on_load)");
  const int64_t ovox = (int64_t)in_size[0] * ksize[0] * in_size[1] * ksize[1] * in_size[2] * ksize[2];
  require(ovox * cout < (1LL << 31), "transposed-convolution output item too large");
  a.ntn = (int)ceil_div(a.ncols, kTcCols);
  require(a.nblk >= a.ntn * (kTcCols / 16), "transposed-convolution packing too small");
  // row tiles per workgroup: up to 16 while the grid keeps >= 2048 workgroups
  const int64_t mtiles = ceil_div(a.M, kTcRows);
  a.tpb = (int)std::max<int64_t>(1, std::min<int64_t>(16, mtiles * a.ntn / 2048));
  const int64_t nwg = ceil_div(mtiles, a.tpb) * a.ntn;
  require(nwg < (1LL << 31), "transposed-convolution grid too large");
  a.nwg = (int)nwg;
  const size_t lds_bytes = (size_t)kTcRows * kTcTileStride * 4 + kTcRows * 8 + kTcCols * 4;
  ProfScope prof(arith == kBf16 ? "tconv3d_x3_bf16" : "tconv3d_x3",
                 2.0 * (double)a.M * cin * a.ncols,
                 4.0 * ((double)a.M * (cin + a.ncols) + (double)cin * a.ncols), st);
  // weights held in registers for up to 2 k-steps (C_in <= 64); more would cost occupancy
  const bool kreg = a.ksteps <= 2;
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(a.nwg), dim3(256), lds_bytes, st, a);
  };
  if (arith == kBf16)
    kreg ? launch(tconv_x3_kernel<kBf16, 2>) : launch(tconv_x3_kernel<kBf16, 0>);
  else
    kreg ? launch(tconv_x3_kernel<kSplit3, 2>) : launch(tconv_x3_kernel<kSplit3, 0>);
  launch_check("tconv3d_split");
}

void conv1x1(const float* x, int cin, const float* w, const float* bias, float* y, int64_t voxels,
             int cout, hipStream_t st, const PendingNorm& nx, int64_t item_voxels) {
  require(x && w && y, "1x1 convolution pointers must not be null");
  require(!nx.params || (item_voxels >= 1 && voxels % item_voxels == 0),
          "a pending normalisation needs the voxels per batch item");
  const int64_t item = nx.params ? item_voxels : 1;
  const int act = nx.act ? 1 : 0;
  require(cin >= 1 && cout >= 1 && (int64_t)cin * cout <= 16384,
          "1x1 convolution weight too large for the head kernel");
  require(voxels >= 1, "empty 1x1 convolution input");
  ProfScope prof("conv1x1_head", 2.0 * (double)voxels * cin * cout, 4.0 * (double)voxels * (cin + cout), st);
  const size_t staged = ((size_t)256 * (cin + 4) + 256 * cout) * sizeof(float);
  const dim3 grid((unsigned)ceil_div(voxels, 256));
  if (cin % 4 == 0 && cin <= 64 && staged <= 96 * 1024) {
    switch (cin / 4) {
#define NNX_HEAD_CASE(Q)                                                                        \
  case Q:                                                                                       \
    hipLaunchKernelGGL(conv1x1_staged_kernel<4 * Q>, grid, dim3(256), staged, st, x, w, bias, y, \
                       voxels, cout, nx.params, act, nx.slope, item);                           \
    break;
      NNX_HEAD_CASE(1) NNX_HEAD_CASE(2) NNX_HEAD_CASE(3) NNX_HEAD_CASE(4)
      NNX_HEAD_CASE(5) NNX_HEAD_CASE(6) NNX_HEAD_CASE(7) NNX_HEAD_CASE(8)
      NNX_HEAD_CASE(9) NNX_HEAD_CASE(10) NNX_HEAD_CASE(11) NNX_HEAD_CASE(12)
      NNX_HEAD_CASE(13) NNX_HEAD_CASE(14) NNX_HEAD_CASE(15) NNX_HEAD_CASE(16)
#undef NNX_HEAD_CASE
    }
  } else
    hipLaunchKernelGGL(conv1x1_kernel, dim3((unsigned)ceil_div(voxels, 256)), dim3(256),
                       (size_t)cin * cout * sizeof(float), st, x, w, bias, y, voxels, cin, cout,
                       nx.params, act, nx.slope, item);
  launch_check("conv1x1");
}

}  // namespace nnx
