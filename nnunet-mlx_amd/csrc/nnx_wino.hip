// Winograd F(2x2x2, 3x3x3) convolution for the stride-1, padding-1 3x3x3 layers, with
// split-fp16 products (hi*hi + hi*lo + lo*hi, float32 accumulation) on
// v_mfma_f32_32x32x16_f16.
//
// A 2x2x2 output tile is Y = A^T [ U (.) V ] A along each axis, with V = B^T d B the
// transform of the tile's 4x4x4 input patch and U = G w G^T the transform of the 3x3x3
// filter (F(2,3): B^T = [1 0 -1 0; 0 1 1 0; 0 -1 1 0; 0 1 0 -1], G = [1 0 0; .5 .5 .5;
// .5 -.5 .5; 0 0 1], A^T = [1 1 1 0; 0 1 -1 -1]).  Summed over input channels, each of the
// 64 transform positions xi = (xz, xy, xx) is an independent GEMM M[xi] = V[xi] U[xi]
// (tiles x C_in times C_in x C_out): 64 products per 8 outputs instead of 216, so the
// three split products cost fewer MFMA operations than one product of the direct
// convolution.  The transforms are exact additions/subtractions of float32 values (and
// the 1/2 of G, exact), so the arithmetic stays float32-class; U is formed in float64 and
// rounded once, V in float32, each then split into fp16 halves.
//
// Workgroup: 8 waves (two a SIMD), an output box of 4 x 8 x 8 voxels (2 x 4 x 4 tiles, the 32
// MFMA rows) of one batch item, and 32 output channels (the 32 MFMA columns).  Wave
// w = 2 xz + p owns the 8 transform positions (xz, xy = 2p or 2p + 1, xx = 0..3): its
// accumulators are 8 blocks of 32 x 32 floats (128 registers a lane), which leaves room for
// a second wave on the SIMD to issue while one waits.  Per chunk of 16 input channels:
//   1. the raw 6 x 10 x 10 input halo was fetched by global_load_lds_dwordx4 into one of two
//      LDS buffers during the previous chunk;
//   2. 400 threads apply the pending InstanceNorm (+ LeakyReLU) of the input to in-volume
//      voxels (inputs without one, such as the transposed convolution's output in a decoder
//      convolution, skip it) and write the z-transform (4 xz x 2 tile rows of z) as 8 padded planes, laid
//      out so that the 32 tiles of a half-wave read 32 different 16-byte bank groups; then
//      the next chunk's halo DMA is issued;
//   3. per y-row of its positions, each wave reads two z-transformed rows of its tile patch,
//      forms V (y- then x-transform), splits it into fp16 halves in registers and issues
//      three MFMAs per position against the packed U of this chunk, read from L2 four
//      positions ahead.
// Epilogue: each wave applies the x- and y-output transforms to its accumulators, the eight
// partials are combined through LDS (z-output transform), scaled back, + bias, written to
// an LDS tile for the InstanceNorm partials of the box and stored as 16-byte channel runs.
#include <cmath>
#include <cstdlib>
#include <string>
#include <type_traits>

#include "nnx_internal.h"

namespace nnx {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

constexpr int kWThreads = 512;                    // 8 waves, two a SIMD
constexpr int kSteps = 8;                         // transform positions (steps) per wave
constexpr int kRing = 4;                          // B operands of four steps in flight
constexpr int kWChunk = 16;                       // input channels per chunk (one MFMA K)
constexpr int kHaloVox = 6 * 10 * 10;             // input halo of a 4 x 8 x 8 output box
constexpr int kRawLines = kHaloVox * 4;           // 16-byte lines (4 channels each)
constexpr int kRawRounds = (kRawLines + kWThreads - 1) / kWThreads;
constexpr int kRawSlots = kRawRounds * kWThreads;  // 16-byte slots per raw buffer
constexpr int kZRow = 41;                          // slots per z-plane row: 10 voxels x 4 + 1
constexpr int kZPlane = 411;                       // slots per plane: 10 rows + 1 slot
constexpr int kZSlots = 8 * kZPlane;
constexpr int kMaxChannels = 1024;                 // c1 + c2 (pending-norm parameters in LDS)
constexpr int kTileStride = 36;                    // floats per voxel row of the output tile
// epilogue: 8 waves x 32 tiles x 32 columns of partials over the raw and z arrays, then the
// output tile + reduction in the raw array
static_assert(8 * 32 * 32 <= 2 * kRawSlots + kZSlots, "epilogue partials fit the main LDS");
static_assert(256 * kTileStride / 4 + kWThreads / 4 <= 2 * kRawSlots, "output tile fits");

struct WinoArgs {
  const float* x0;
  const float* x1;
  int c0, c1, chunks0, chunks;
  const uint4* u;  // packed transformed weights
  const float* bias;
  float* y;
  int D, H, W;
  int cout, ntn;
  int nbz, nby, nbx;
  int nwg;
  int nbox;   // batch * nbz * nby * nbx (boxes of one column block)
  int nvirt;  // nbox * ntn: (column block, box) pairs, column block slowest
  float out_scale;
  float4* stats;
  const float4* nrm0;
  const float4* nrm1;
  int act0, act1;
  float slope;
};

// 16 zero bytes: halo lines outside the volume are fetched from here.
__device__ __align__(16) float g_wino_zero[4];

__device__ __forceinline__ f16v mfma32(h8 a, h8 b, f16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// hi = fp16(v) (nearest even), lo = fp16(v - hi).  v - hi is exact in float32, so the
// single rounding of v_fma_mix{lo,hi}_f16 (fma(-hi, 1, v) formed exactly, rounded once to
// fp16) gives the same lo as converting hi back, subtracting and converting: one
// instruction per element instead of three.
__device__ __forceinline__ void split8(const float (&v)[8], h8& hi, h8& lo) {
#pragma unroll
  for (int q = 0; q < 8; q += 2) {
    const h2 h = __builtin_convertvector((f2{v[q], v[q + 1]}), h2);
    h2 l;
    asm("v_fma_mixlo_f16 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(l) : "v"(h), "v"(v[q]));
    asm("v_fma_mixhi_f16 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "+v"(l) : "v"(h), "v"(v[q + 1]));
    hi[q] = h[0];
    hi[q + 1] = h[1];
    lo[q] = l[0];
    lo[q + 1] = l[1];
  }
}

// Two z-plane rows of a tile patch (4 columns x 2 channel halves each, 16 B per read) at LDS
// byte offsets a and b, with the wait for them.  Written as one asm block so that the
// compiler's wait-count pass does not see LDS reads here: it would otherwise order them
// behind the halo DMA issued just before into another buffer (it cannot tell the two apart)
// and wait for that DMA first.
__device__ __forceinline__ void zrow_pair(unsigned a, unsigned b, f4 (&va)[8], f4 (&vb)[8]) {
  asm volatile(
      "ds_read_b128 %0, %16\n\tds_read_b128 %1, %16 offset:16\n\t"
      "ds_read_b128 %2, %16 offset:64\n\tds_read_b128 %3, %16 offset:80\n\t"
      "ds_read_b128 %4, %16 offset:128\n\tds_read_b128 %5, %16 offset:144\n\t"
      "ds_read_b128 %6, %16 offset:192\n\tds_read_b128 %7, %16 offset:208\n\t"
      "ds_read_b128 %8, %17\n\tds_read_b128 %9, %17 offset:16\n\t"
      "ds_read_b128 %10, %17 offset:64\n\tds_read_b128 %11, %17 offset:80\n\t"
      "ds_read_b128 %12, %17 offset:128\n\tds_read_b128 %13, %17 offset:144\n\t"
      "ds_read_b128 %14, %17 offset:192\n\tds_read_b128 %15, %17 offset:208\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(va[0]), "=&v"(va[1]), "=&v"(va[2]), "=&v"(va[3]), "=&v"(va[4]), "=&v"(va[5]),
        "=&v"(va[6]), "=&v"(va[7]), "=&v"(vb[0]), "=&v"(vb[1]), "=&v"(vb[2]), "=&v"(vb[3]),
        "=&v"(vb[4]), "=&v"(vb[5]), "=&v"(vb[6]), "=&v"(vb[7])
      : "v"(a), "v"(b)
      : "memory");
}

// For lanes 0-31: x + (lane + 32's x), by v_permlane32_swap (lanes 32-63 of the first
// operand trade places with lanes 0-31 of the second) instead of an LDS permute.  Lanes
// 32-63 get x + x (unused).
__device__ __forceinline__ float add_upper_half(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return x + __uint_as_float(r[1]);
}

// The InstanceNorm apply pass's operations: r = fma(x - mean, scale, beta), then
// max(s * r, r) with s = the LeakyReLU slope under the activation and s = 1 (the identity,
// exactly) without it.
__device__ __forceinline__ f4 wino_norm(f4 v, const float4 (&p)[4], float s) {
  f4 r;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float t = fmaf(v[q] - p[q].x, p[q].y, p[q].z);
    r[q] = fmaxf(s * t, t);
  }
  return r;
}

__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// The end of a box's epilogue, shared by both kernels.  yo[k][oz] holds, for column
// c = tid % 32 and tile (tid / 32) + 16 k of the box, the four (oy, ox) outputs of z output
// oz.  The values go to the output tile in LDS (row per box voxel, stride kTileStride) and
// leave as 16-byte channel runs; the box's InstanceNorm partials per column (mean over the
// valid voxels, then the centred sum of squares) are reduced from the registers: a thread's
// 16 voxels, the two lanes of a wave holding the column, then the eight waves through the
// two 256-float arrays after the tile.  Barriers wait for LDS only.  kFull: the box lies
// wholly inside the volume (no per-voxel checks).
template <bool kFull>
__device__ __forceinline__ void wino_epilogue_tail_t(const WinoArgs& a, const f4 (&yo)[2][2],
                                                     float* otile, int tid, int lane, int wave,
                                                     int b, int nt, int bzi, int byi, int bxi) {
  const int oz0 = bzi * 4, oy0 = byi * 8, ox0 = bxi * 8;
  const int c = tid & 31;
  auto voxel = [&](int k, int oz, int e) {
    const int tile = (tid >> 5) + 16 * k;
    const int tz = tile >> 4, ty = (tile >> 2) & 3, tx = tile & 3;
    return ((2 * tz + oz) * 8 + 2 * ty + (e >> 1)) * 8 + 2 * tx + (e & 1);
  };
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int oz = 0; oz < 2; ++oz)
#pragma unroll
      for (int e = 0; e < 4; ++e) otile[voxel(k, oz, e) * kTileStride + c] = yo[k][oz][e];
  auto valid = [&](int v) {
    return oz0 + (v >> 6) < a.D && oy0 + ((v >> 3) & 7) < a.H && ox0 + (v & 7) < a.W;
  };
  float* red = otile + 256 * kTileStride;  // [wave][column] sums, then centred squares
  const int nz = min(4, a.D - oz0), ny = min(8, a.H - oy0), nx = min(8, a.W - ox0);
  const float cnt = (float)(nz * ny * nx);
  if (a.stats) {
    float sm = 0.f;
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int oz = 0; oz < 2; ++oz)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (kFull || valid(voxel(k, oz, e))) sm += yo[k][oz][e];
    sm = add_upper_half(sm);
    if (lane < 32) red[wave * 32 + c] = sm;
  }
  lds_barrier();  // the tile and the sums
  if (a.stats) {
    // the eight waves' sums read together, then added in wave order
    float rv[kWThreads / 64];
#pragma unroll
    for (int w = 0; w < kWThreads / 64; ++w) rv[w] = red[w * 32 + c];
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kWThreads / 64; ++w) tot += rv[w];
    const float mean = tot / cnt;
    float m2 = 0.f;
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int oz = 0; oz < 2; ++oz)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (kFull || valid(voxel(k, oz, e))) {
            const float d = yo[k][oz][e] - mean;
            m2 = fmaf(d, d, m2);
          }
    m2 = add_upper_half(m2);
    if (lane < 32) red[256 + wave * 32 + c] = m2;
    lds_barrier();
    if (tid < 32) {
#pragma unroll
      for (int w = 0; w < kWThreads / 64; ++w) rv[w] = red[256 + w * 32 + c];
      float tm = 0.f;
#pragma unroll
      for (int w = 0; w < kWThreads / 64; ++w) tm += rv[w];
      const int tiles = a.nbz * a.nby * a.nbx;
      const int tile_s = (bzi * a.nby + byi) * a.nbx + bxi;
      a.stats[((int64_t)b * tiles + tile_s) * a.cout + nt * 32 + c] = make_float4(mean, tm, cnt, 0.f);
    }
  }
  // stores: 256 voxels x 8 runs of 4 channels; thread tid stores run tid % 8 of voxel
  // (z, y, x) = (k, (tid / 64) % 8, (tid / 8) % 8) of the box in round k, so only z moves
  // between its rounds (one 64-bit address, then a plane stride)
  const int qd = tid & 7, vyx = (tid >> 3) & 63;
  const int yy = oy0 + (vyx >> 3), xx = ox0 + (vyx & 7);
  const int64_t base =
      (((int64_t)b * a.D + oz0) * a.H * a.W + (int64_t)yy * a.W + xx) * a.cout + nt * 32 + 4 * qd;
  const int64_t zstride = (int64_t)a.H * a.W * a.cout;
  static_assert(256 * 8 / kWThreads == 4 && kWThreads == 512, "one box z-plane a round");
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int v = k * 64 + vyx;
    if (kFull || valid(v)) {
      const float* src = otile + v * kTileStride + 4 * qd;
      *reinterpret_cast<f4*>(a.y + base + k * zstride) = f4{src[0], src[1], src[2], src[3]};
    }
  }
}

__device__ __forceinline__ void wino_epilogue_tail(const WinoArgs& a, const f4 (&yo)[2][2],
                                                   float* otile, int tid, int lane, int wave,
                                                   int b, int nt, int bzi, int byi, int bxi) {
  // uniform over the workgroup
  if (bzi * 4 + 4 <= a.D && byi * 8 + 8 <= a.H && bxi * 8 + 8 <= a.W)
    wino_epilogue_tail_t<true>(a, yo, otile, tid, lane, wave, b, nt, bzi, byi, bxi);
  else
    wino_epilogue_tail_t<false>(a, yo, otile, tid, lane, wave, b, nt, bzi, byi, bxi);
}

__global__ __launch_bounds__(kWThreads, 1) void wino_x3_kernel(WinoArgs a) {
  // three LDS objects: the compiler then knows that the halo DMA into s_raw does not write
  // what the later reads of s_prm read
  __shared__ __align__(16) f4 s_raw[2 * kRawSlots];  // two raw halo buffers
  __shared__ __align__(16) f4 s_z[kZSlots];          // z-transformed planes
  __shared__ __align__(16) f4 s_prm[kMaxChannels];   // pending-norm parameters
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int logical = xcd_remap(blockIdx.x, a.nwg);
  const int nt = logical % a.ntn;
  int box = logical / a.ntn;
  const int bxi = box % a.nbx;
  box /= a.nbx;
  const int byi = box % a.nby;
  box /= a.nby;
  const int bzi = box % a.nbz;
  const int b = box / a.nbz;
  const int oz0 = bzi * 4, oy0 = byi * 8, ox0 = bxi * 8;
  const int iz0 = oz0 - 1, iy0 = oy0 - 1, ix0 = ox0 - 1;
  const int64_t bvox = (int64_t)b * a.D * a.H * a.W;

  // ---- raw halo fetch of one chunk into buffer `buf` (LDS slot = line = voxel * 4 + quad);
  // this thread's lines r * kWThreads + tid have fixed voxels: their offsets inside the batch
  // item (-1 outside the volume or past the halo) are computed once
  const int cq_line = tid & 3;
  int vofs[kRawRounds];
#pragma unroll
  for (int r = 0; r < kRawRounds; ++r) {
    const int line = r * kWThreads + tid;
    int o = -1;
    if (line < kRawLines) {
      const int v = line >> 2;
      const int hz = v / 100, rem = v - hz * 100;
      const int hy = rem / 10, hx = rem - hy * 10;
      const int z = iz0 + hz, yy = iy0 + hy, xx = ix0 + hx;
      if ((unsigned)z < (unsigned)a.D && (unsigned)yy < (unsigned)a.H &&
          (unsigned)xx < (unsigned)a.W)
        o = (z * a.H + yy) * a.W + xx;
    }
    vofs[r] = o;
  }
  // past the last chunk (live = false) every line reads the zero line: the DMA is issued
  // unconditionally, so no branch joins paths with different counts of loads in flight
  auto fetch = [&](int chunk, int buf, bool live) __attribute__((always_inline)) {
    const bool first = chunk < a.chunks0;
    const float* src = first ? a.x0 : a.x1;
    const int C = first ? a.c0 : a.c1;
    const float* base = src + bvox * C + (first ? chunk : chunk - a.chunks0) * kWChunk + cq_line * 4;
    f4* dst = s_raw + buf * kRawSlots + wave * 64;
#pragma unroll
    for (int r = 0; r < kRawRounds; ++r) {
      // both addresses formed and one selected: no branch around the load, so the
      // compiler's wait counts stay exact
      const float* in = base + (int64_t)(vofs[r] < 0 ? 0 : vofs[r]) * C;
      const float* g = live && vofs[r] >= 0 ? in : g_wino_zero;
      __builtin_amdgcn_global_load_lds(
          g, (__attribute__((address_space(3))) void*)(dst + r * kWThreads), 16, 0, 0);
    }
  };

  // ---- pending InstanceNorm parameters of every input channel (both inputs, in chunk
  // order) for this batch item
  for (int c = tid; c < a.c0 + a.c1; c += kWThreads) {
    const float4* pp = c < a.c0 ? a.nrm0 : a.nrm1;
    const int C = c < a.c0 ? a.c0 : a.c1;
    const int cc = c < a.c0 ? c : c - a.c0;
    float4 v = make_float4(0.f, 1.f, 0.f, 0.f);
    if (pp) v = pp[(int64_t)b * C + cc];
    s_prm[c] = f4{v.x, v.y, v.z, 0.f};
  }

  // ---- pending norm + z-transform: thread (hy, hx, quad) of the 10 x 10 x 4 columns.  A
  // halo wholly inside the volume (uniform over the workgroup) needs no padding selects.
  const bool interior = iz0 >= 0 && iz0 + 6 <= a.D && iy0 >= 0 && iy0 + 10 <= a.H &&
                        ix0 >= 0 && ix0 + 10 <= a.W;
  auto transform_column = [&](auto inner, int chunk, int buf, int col) __attribute__((always_inline)) {
    const int hy = col / 40, rem = col - hy * 40;
    const int hx = rem >> 2, cq = rem & 3;
    const bool first = chunk < a.chunks0;
    const float s = (first ? a.act0 : a.act1) != 0 ? a.slope : 1.f;
    // parameters of inputs without a pending norm are (0, 1, 0): the identity
    float4 pm[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f4 v = s_prm[chunk * kWChunk + cq * 4 + q];
      pm[q] = make_float4(v[0], v[1], v[2], 0.f);
    }
    const f4* raw = s_raw + buf * kRawSlots + (hy * 10 + hx) * 4 + cq;
    f4 d[6];
#pragma unroll
    for (int hz = 0; hz < 6; ++hz) d[hz] = raw[hz * 400];
    if constexpr (decltype(inner)::value == 2) {
      // no pending norm: the raw values (the padding lines read the zero line)
    } else if constexpr (decltype(inner)::value == 1) {
#pragma unroll
      for (int hz = 0; hz < 6; ++hz) d[hz] = wino_norm(d[hz], pm, s);
    } else {
      const bool inyx =
          (unsigned)(iy0 + hy) < (unsigned)a.H && (unsigned)(ix0 + hx) < (unsigned)a.W;
#pragma unroll
      for (int hz = 0; hz < 6; ++hz) {
        // the padding stays zero; in-volume voxels take the pending norm
        const f4 t = wino_norm(d[hz], pm, s);
        const bool inside = inyx && (unsigned)(iz0 + hz) < (unsigned)a.D;
#pragma unroll
        for (int e = 0; e < 4; ++e) d[hz][e] = inside ? t[e] : 0.f;
      }
    }
    f4* dst = s_z + hy * kZRow + hx * 4 + cq;
#pragma unroll
    for (int tz = 0; tz < 2; ++tz) {
      const f4 d0 = d[2 * tz], d1 = d[2 * tz + 1], d2 = d[2 * tz + 2], d3 = d[2 * tz + 3];
      dst[(0 * 2 + tz) * kZPlane] = d0 - d2;
      dst[(1 * 2 + tz) * kZPlane] = d1 + d2;
      dst[(2 * 2 + tz) * kZPlane] = d2 - d1;
      dst[(3 * 2 + tz) * kZPlane] = d1 - d3;
    }
  };
  auto transform = [&](int chunk, int buf) __attribute__((always_inline)) {
    if (tid < 400) {
      if ((chunk < a.chunks0 ? a.nrm0 : a.nrm1) == nullptr)
        transform_column(std::integral_constant<int, 2>{}, chunk, buf, tid);
      else if (interior)
        transform_column(std::integral_constant<int, 1>{}, chunk, buf, tid);
      else
        transform_column(std::integral_constant<int, 0>{}, chunk, buf, tid);
    }
  };

  // ---- this lane's tile, channel half and transform positions: wave = (xz, half p), the
  // half owning xy = 2p and 2p + 1
  const int xz = wave >> 1, p = wave & 1;
  const int t = lane & 31, tzl = t >> 4, tyl = (t >> 2) & 3, txl = t & 3, g8 = lane >> 5;
  // LDS byte offset of this lane's first z-row read (tile patch corner, channel half g8)
  const unsigned zb_lds = (unsigned)(uintptr_t)(
      (__attribute__((address_space(3))) f4*)s_z + ((xz * 2 + tzl) * kZPlane + (2 * tyl) * kZRow +
                                                    (2 * txl) * 4 + 2 * g8));

  // packed U: [nt][chunk][xi = (xz * 4 + xy) * 4 + xx][hi | lo][64 lanes] x 16 bytes; step
  // s (local xy = s / 4, xx = s % 4) of a chunk uses position xi = xz * 16 + p * 8 + s
  const uint4* ub = a.u + ((int64_t)nt * a.chunks * 64 + xz * 16 + p * kSteps) * 128 + lane;
  auto uaddr = [&](int chunk, int step) { return ub + ((int64_t)chunk * 64 + step) * 128; };

  f16v acc[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][x][r] = 0.f;

  uint4 uh[kRing], ul[kRing];
  fetch(0, 0, true);
#pragma unroll
  for (int s = 0; s < kRing; ++s) {
    const uint4* up = uaddr(0, s);
    uh[s] = up[0];
    ul[s] = up[64];
  }

  // the three products of step s (local xy = s / 4, xx = s % 4) for two steps at a time,
  // then the refill of their ring slots kRing steps ahead
  auto products = [&](int s0, const float (&q)[4][8], int chunk) __attribute__((always_inline)) {
    h8 ah[2], al[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int xx = (s0 + k) & 3;
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (xx == 0) v[e] = q[0][e] - q[2][e];
        else if (xx == 1) v[e] = q[1][e] + q[2][e];
        else if (xx == 2) v[e] = q[2][e] - q[1][e];
        else v[e] = q[1][e] - q[3][e];
      }
      split8(v, ah[k], al[k]);
    }
    const int xy = s0 >> 2, x0 = s0 & 3;
#pragma unroll
    for (int k = 0; k < 2; ++k)
      acc[xy][x0 + k] = mfma32(ah[k], *reinterpret_cast<const h8*>(&uh[(s0 + k) % kRing]),
                               acc[xy][x0 + k]);
#pragma unroll
    for (int k = 0; k < 2; ++k)
      acc[xy][x0 + k] = mfma32(ah[k], *reinterpret_cast<const h8*>(&ul[(s0 + k) % kRing]),
                               acc[xy][x0 + k]);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int s = s0 + k, slot = s % kRing;
      acc[xy][x0 + k] = mfma32(al[k], *reinterpret_cast<const h8*>(&uh[slot]), acc[xy][x0 + k]);
      // unconditional (past the last chunk the last chunk's words are read again)
      const int ns = s + kRing;
      int nchunk = ns < kSteps ? chunk : chunk + 1;
      nchunk = nchunk < a.chunks ? nchunk : a.chunks - 1;
      const uint4* up = uaddr(nchunk, ns & (kSteps - 1));
      uh[slot] = up[0];
      ul[slot] = up[64];
    }
  };

  // one y-row of Q at a time: half 0 forms xy 0, 1 (r0 - r2, r1 + r2), half 1 xy 2, 3
  // (r2 - r1, r1 - r3), i.e. Q0 = R[2p] - R[2 - p] and Q1 = R[1] + sg R[2 + p] with sg = +-1
  // (fma: one rounding, as the add or subtract)
  const float sg = p ? -1.f : 1.f;
  // the host launches only layers with input channels (chunks >= 1): without this the
  // compiler keeps a zeroed copy of the accumulators for the loop-skipping path as well
  __builtin_assume(a.chunks > 0);
  for (int chunk = 0; chunk < a.chunks; ++chunk) {
    const int buf = chunk & 1;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's halo lines and B operands have landed
    __syncthreads();                 // every thread's; the z-planes are free
    transform(chunk, buf);
    // the next chunk's halo into the other buffer (free since this chunk began), after this
    // thread's reads of `buf`: a whole chunk of products covers its latency
    const bool more = chunk + 1 < a.chunks;
    fetch(more ? chunk + 1 : chunk, buf ^ 1, more);
    // z-planes written: this thread's LDS writes complete, then the barrier.  Not
    // __syncthreads(), whose release fence would also wait for the DMA just issued (nothing
    // reads that buffer before the next chunk's full wait and barrier).
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f4 va[8], vb[8];  // [column * 2 + half]
      zrow_pair(zb_lds + (j == 0 ? 2 * p : 1) * kZRow * 16,
                zb_lds + (j == 0 ? 2 - p : 2 + p) * kZRow * 16, va, vb);
      float q[4][8];
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            q[c][4 * h + e] = j == 0 ? va[2 * c + h][e] - vb[2 * c + h][e]
                                     : fmaf(sg, vb[2 * c + h][e], va[2 * c + h][e]);
      products(4 * j, q, chunk);
      products(4 * j + 2, q, chunk);
    }
  }

  // ---- epilogue
  // x- and y-output transforms of this wave's positions: per accumulator element, this
  // half's share of the (oy, ox) outputs of its tile row for this xz (oy0 = xy0 + xy1 +
  // xy2, oy1 = xy1 - xy2 - xy3)
  __builtin_amdgcn_s_waitcnt(0);  // the last (zero-line) DMA has landed in s_raw
  __syncthreads();                 // every wave is past its last z-plane read and DMA
  // partials [wave][tile][column] x (oy0ox0, oy0ox1, oy1ox0, oy1ox1): waves 0-4 in s_raw,
  // waves 5-7 in s_z
  auto part = [&](int w, int tile, int c) -> f4& {
    const int i = (w * 32 + tile) * 32 + c;
    return i < 2 * kRawSlots ? s_raw[i] : s_z[i - 2 * kRawSlots];
  };
  const int col = lane & 31;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float xo[2][2];  // [local xy][ox]
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float m0 = acc[j][0][r], m1 = acc[j][1][r], m2 = acc[j][2][r], m3 = acc[j][3][r];
      xo[j][0] = (m0 + m1) + m2;
      xo[j][1] = (m1 - m2) - m3;
    }
    const f4 pv = p == 0 ? f4{xo[0][0] + xo[1][0], xo[0][1] + xo[1][1], xo[1][0], xo[1][1]}
                         : f4{xo[0][0], xo[0][1], -(xo[0][0] + xo[1][0]), -(xo[0][1] + xo[1][1])};
    const int tile = 8 * (r >> 2) + 4 * g8 + (r & 3);
    part(wave, tile, col) = pv;
  }
  __syncthreads();
  // z-output transform over the four xz partials: oz0 = P0 + P1 + P2, oz1 = P1 - P2 - P3;
  // then the weight scale and the bias
  constexpr int kPairs = 32 * 32 / kWThreads;
  f4 yo[kPairs][2];  // [pair][oz]
  const float bias_c = a.bias ? a.bias[nt * 32 + (tid & 31)] : 0.f;
#pragma unroll
  for (int k = 0; k < kPairs; ++k) {
    const int idx = tid + k * kWThreads;
    const int tile = idx >> 5, c = idx & 31;
    f4 pz[4];
#pragma unroll
    for (int z = 0; z < 4; ++z) pz[z] = part(2 * z, tile, c) + part(2 * z + 1, tile, c);
    const f4 y0 = (pz[0] + pz[1]) + pz[2];
    const f4 y1 = (pz[1] - pz[2]) - pz[3];
    yo[k][0] = y0 * a.out_scale;
    yo[k][1] = y1 * a.out_scale;
    if (a.bias) {
      yo[k][0] = yo[k][0] + bias_c;
      yo[k][1] = yo[k][1] + bias_c;
    }
  }
  __syncthreads();  // every thread's partial reads are done: the tile may overwrite them
  wino_epilogue_tail(a, yo, reinterpret_cast<float*>(s_raw), tid, lane, wave, b, nt, bzi, byi,
                     bxi);
}

// ---- persistent variant ------------------------------------------------------------
// One workgroup a CU loops over boxes.  The eight XCDs take contiguous ranges of the
// (column block, box) pairs, column block slowest, and the G workgroups of an XCD interleave
// over its range, so an XCD's L2 holds one column block's packed weights and neighbouring
// boxes' halos.  The box arithmetic is the kernel above's, in the same order (the results
// are bit-identical); what changes is the overlap between boxes: the last chunk of a box
// issues the next box's first halo DMA and its B-operand refills load the next box's first
// four steps, so the next box starts with its halo and weights landed instead of waiting for
// them (~8k cycles a box).  The epilogue therefore keeps out of the raw halo buffers (its
// partials, two rounds of 16 tiles, and its output tile live in the z-planes and the
// parameter table, whose next box's values are loaded after it), its barriers wait for LDS
// only, and the bias is read at box start.
struct WinoBox {
  int nt, b, bzi, byi, bxi;
};

__device__ __forceinline__ WinoBox wino_box(const WinoArgs& a, int v) {
  WinoBox r;
  r.nt = v / a.nbox;
  int box = v - r.nt * a.nbox;
  r.bxi = box % a.nbx;
  box /= a.nbx;
  r.byi = box % a.nby;
  box /= a.nby;
  r.bzi = box % a.nbz;
  r.b = box / a.nbz;
  return r;
}


__global__ __launch_bounds__(kWThreads, 1) void wino_x3p_kernel(WinoArgs a) {
  __shared__ __align__(16) f4 s_raw[2 * kRawSlots];  // two raw halo buffers
  __shared__ __align__(16) f4 s_z[kZSlots];          // z-planes; epilogue partials and tile
  __shared__ __align__(16) f4 s_prm[kMaxChannels];   // parameters; epilogue partials
  // the bias of the current box's column block (read in the epilogue from LDS: a global
  // read there would wait for the next box's halo DMA)
  __shared__ float s_bias[32];
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  // this workgroup's (column block, box) pairs: XCD blockIdx % 8 takes a contiguous range,
  // its G workgroups interleave over it (the grid is a multiple of 8)
  const int xcd = blockIdx.x & 7, G = gridDim.x >> 3;
  const int vq = a.nvirt >> 3, vr = a.nvirt & 7;
  const int vbeg = xcd < vr ? xcd * (vq + 1) : vr * (vq + 1) + (xcd - vr) * vq;
  const int vend = vbeg + vq + (xcd < vr ? 1 : 0);
  int v = vbeg + (int)(blockIdx.x >> 3);
  if (v >= vend) return;  // uniform over the workgroup, before any barrier
  const int xz = wave >> 1, p = wave & 1;
  const float sg = p ? -1.f : 1.f;
  __builtin_assume(a.chunks > 0);
  constexpr int kPairs = 32 * 32 / kWThreads;

  // halo line offsets of a box inside its batch item (-1 outside the volume or the halo)
  auto box_vofs = [&](int tid, const WinoBox& bx, int (&vofs)[kRawRounds])
      __attribute__((always_inline)) {
    const int iz0 = bx.bzi * 4 - 1, iy0 = bx.byi * 8 - 1, ix0 = bx.bxi * 8 - 1;
#pragma unroll
    for (int r = 0; r < kRawRounds; ++r) {
      const int line = r * kWThreads + tid;
      int o = -1;
      if (line < kRawLines) {
        const int hv = line >> 2;
        const int hz = hv / 100, rem = hv - hz * 100;
        const int hy = rem / 10, hx = rem - hy * 10;
        const int z = iz0 + hz, yy = iy0 + hy, xx = ix0 + hx;
        if ((unsigned)z < (unsigned)a.D && (unsigned)yy < (unsigned)a.H &&
            (unsigned)xx < (unsigned)a.W)
          o = (z * a.H + yy) * a.W + xx;
      }
      vofs[r] = o;
    }
  };
  // chunk `chunk` of item b's halo lines into buffer `buf` (live = false: the zero line)
  auto fetch = [&](int tid, int b, const int (&vofs)[kRawRounds], int chunk, int buf, bool live)
      __attribute__((always_inline)) {
    const bool first = chunk < a.chunks0;
    const float* src = first ? a.x0 : a.x1;
    const int C = first ? a.c0 : a.c1;
    const int64_t bv = (int64_t)b * a.D * a.H * a.W;
    const float* base = src + bv * C + (first ? chunk : chunk - a.chunks0) * kWChunk + (tid & 3) * 4;
    f4* dst = s_raw + buf * kRawSlots + wave * 64;
#pragma unroll
    for (int r = 0; r < kRawRounds; ++r) {
      const float* in = base + (int64_t)(vofs[r] < 0 ? 0 : vofs[r]) * C;
      const float* g = live && vofs[r] >= 0 ? in : g_wino_zero;
      __builtin_amdgcn_global_load_lds(
          g, (__attribute__((address_space(3))) void*)(dst + r * kWThreads), 16, 0, 0);
    }
  };
  auto load_prm = [&](int tid, int b) __attribute__((always_inline)) {
    for (int c = tid; c < a.c0 + a.c1; c += kWThreads) {
      const float4* pp = c < a.c0 ? a.nrm0 : a.nrm1;
      const int C = c < a.c0 ? a.c0 : a.c1;
      const int cc = c < a.c0 ? c : c - a.c0;
      float4 pv = make_float4(0.f, 1.f, 0.f, 0.f);
      if (pp) pv = pp[(int64_t)b * C + cc];
      s_prm[c] = f4{pv.x, pv.y, pv.z, 0.f};
    }
  };
  // packed U words of column block ntb, chunk, step (local position) for this lane
  auto uaddr = [&](int lane, int ntb, int chunk, int step) {
    return a.u + (((int64_t)ntb * a.chunks + chunk) * 64 + xz * 16 + p * kSteps + step) * 128 + lane;
  };

  // loop-carried state: the halo offsets of the box whose first chunk is in flight, the
  // B-operand ring, the bias of the current column block
  int vofs[kRawRounds];
  uint4 uh[kRing], ul[kRing];
  {
    const int tid = threadIdx.x;
    const WinoBox first = wino_box(a, v);
    box_vofs(tid, first, vofs);
    load_prm(tid, first.b);
    fetch(tid, first.b, vofs, 0, 0, true);
#pragma unroll
    for (int s0 = 0; s0 < kRing; ++s0) {
      const uint4* up = uaddr(tid & 63, first.nt, 0, s0);
      uh[s0] = up[0];
      ul[s0] = up[64];
    }
    if (tid < 32) s_bias[tid] = a.bias ? a.bias[first.nt * 32 + tid] : 0.f;
  }

  for (;;) {
    // per-lane values rebuilt from an opaque copy each box, so that nothing derived from
    // them is hoisted out of the box loop and held through it
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const WinoBox cur = wino_box(a, v);
    const int vnext = v + G;
    const bool more = vnext < vend;
    const int vn = more ? vnext : v;  // the next box (this one again after the last)
    const int nnt = vn / a.nbox;
    const int iz0 = cur.bzi * 4 - 1, iy0 = cur.byi * 8 - 1, ix0 = cur.bxi * 8 - 1;
    const bool interior = iz0 >= 0 && iz0 + 6 <= a.D && iy0 >= 0 && iy0 + 10 <= a.H &&
                          ix0 >= 0 && ix0 + 10 <= a.W;
    const int t = lane & 31, tzl = t >> 4, tyl = (t >> 2) & 3, txl = t & 3, g8 = lane >> 5;
    const unsigned zb_lds = (unsigned)(uintptr_t)(
        (__attribute__((address_space(3))) f4*)s_z + ((xz * 2 + tzl) * kZPlane + (2 * tyl) * kZRow +
                                                      (2 * txl) * 4 + 2 * g8));
    auto transform_column = [&](auto inner, int chunk, int buf, int col)
        __attribute__((always_inline)) {
      const int hy = col / 40, rem = col - hy * 40;
      const int hx = rem >> 2, cq = rem & 3;
      const bool first = chunk < a.chunks0;
      const float sl = (first ? a.act0 : a.act1) != 0 ? a.slope : 1.f;
      float4 pm[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f4 pq = s_prm[chunk * kWChunk + cq * 4 + q];
        pm[q] = make_float4(pq[0], pq[1], pq[2], 0.f);
      }
      const f4* raw = s_raw + buf * kRawSlots + (hy * 10 + hx) * 4 + cq;
      f4 d[6];
#pragma unroll
      for (int hz = 0; hz < 6; ++hz) d[hz] = raw[hz * 400];
      if constexpr (decltype(inner)::value == 2) {
        // no pending norm: the raw values (the padding lines read the zero line)
      } else if constexpr (decltype(inner)::value == 1) {
#pragma unroll
        for (int hz = 0; hz < 6; ++hz) d[hz] = wino_norm(d[hz], pm, sl);
      } else {
        const bool inyx =
            (unsigned)(iy0 + hy) < (unsigned)a.H && (unsigned)(ix0 + hx) < (unsigned)a.W;
#pragma unroll
        for (int hz = 0; hz < 6; ++hz) {
          const f4 tq = wino_norm(d[hz], pm, sl);
          const bool inside = inyx && (unsigned)(iz0 + hz) < (unsigned)a.D;
#pragma unroll
          for (int e = 0; e < 4; ++e) d[hz][e] = inside ? tq[e] : 0.f;
        }
      }
      f4* dst = s_z + hy * kZRow + hx * 4 + cq;
#pragma unroll
      for (int tz = 0; tz < 2; ++tz) {
        const f4 d0 = d[2 * tz], d1 = d[2 * tz + 1], d2 = d[2 * tz + 2], d3 = d[2 * tz + 3];
        dst[(0 * 2 + tz) * kZPlane] = d0 - d2;
        dst[(1 * 2 + tz) * kZPlane] = d1 + d2;
        dst[(2 * 2 + tz) * kZPlane] = d2 - d1;
        dst[(3 * 2 + tz) * kZPlane] = d1 - d3;
      }
    };

    f16v acc[2][4];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[jj][x][r] = 0.f;

    // the three products of steps s0, s0 + 1, then their ring refills kRing steps ahead:
    // past the chunk's last step the next chunk's, past the box's last chunk the next box's
    // first chunk's (column block nnt)
    auto products = [&](int s0, const float (&q)[4][8], int chunk) __attribute__((always_inline)) {
      h8 ah[2], al[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int xx = (s0 + k) & 3;
        float vv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (xx == 0) vv[e] = q[0][e] - q[2][e];
          else if (xx == 1) vv[e] = q[1][e] + q[2][e];
          else if (xx == 2) vv[e] = q[2][e] - q[1][e];
          else vv[e] = q[1][e] - q[3][e];
        }
        split8(vv, ah[k], al[k]);
      }
      const int xy = s0 >> 2, x0 = s0 & 3;
#pragma unroll
      for (int k = 0; k < 2; ++k)
        acc[xy][x0 + k] = mfma32(ah[k], *reinterpret_cast<const h8*>(&uh[(s0 + k) % kRing]),
                                 acc[xy][x0 + k]);
#pragma unroll
      for (int k = 0; k < 2; ++k)
        acc[xy][x0 + k] = mfma32(ah[k], *reinterpret_cast<const h8*>(&ul[(s0 + k) % kRing]),
                                 acc[xy][x0 + k]);
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int st = s0 + k, slot_r = st % kRing;
        acc[xy][x0 + k] = mfma32(al[k], *reinterpret_cast<const h8*>(&uh[slot_r]), acc[xy][x0 + k]);
        const int ns = st + kRing;
        const bool wrap = ns >= kSteps && chunk + 1 >= a.chunks;
        const uint4* up = uaddr(lane, wrap ? nnt : cur.nt,
                                ns < kSteps ? chunk : (wrap ? 0 : chunk + 1), ns & (kSteps - 1));
        uh[slot_r] = up[0];
        ul[slot_r] = up[64];
      }
    };

    for (int chunk = 0; chunk < a.chunks; ++chunk) {
      const int buf = chunk & 1;
      __builtin_amdgcn_s_waitcnt(0);  // this thread's halo lines and B operands have landed
      __syncthreads();                 // every thread's; the z-planes are free
      if (tid < 400) {
        if ((chunk < a.chunks0 ? a.nrm0 : a.nrm1) == nullptr)
          transform_column(std::integral_constant<int, 2>{}, chunk, buf, tid);
        else if (interior)
          transform_column(std::integral_constant<int, 1>{}, chunk, buf, tid);
        else
          transform_column(std::integral_constant<int, 0>{}, chunk, buf, tid);
      }
      // the next chunk's halo into the other buffer; after the box's last chunk the next
      // box's first chunk (the zero line after the last box)
      if (chunk + 1 < a.chunks) {
        fetch(tid, cur.b, vofs, chunk + 1, buf ^ 1, true);
      } else {
        // (from an opaque copy of the thread index: computed here, not hoisted to the box
        // start and held through the chunk loop)
        int tid_n = tid;
        asm volatile("" : "+v"(tid_n));
        const WinoBox nb = wino_box(a, vn);
        box_vofs(tid_n, nb, vofs);
        fetch(tid_n, nb.b, vofs, 0, buf ^ 1, more);
      }
      lds_barrier();
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        f4 va[8], vb[8];
        zrow_pair(zb_lds + (j == 0 ? 2 * p : 1) * kZRow * 16,
                  zb_lds + (j == 0 ? 2 - p : 2 + p) * kZRow * 16, va, vb);
        float q[4][8];
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              q[c][4 * h + e] = j == 0 ? va[2 * c + h][e] - vb[2 * c + h][e]
                                       : fmaf(sg, vb[2 * c + h][e], va[2 * c + h][e]);
        products(4 * j, q, chunk);
        products(4 * j + 2, q, chunk);
      }
    }

    // ---- epilogue in the z-planes and the parameter table only
    lds_barrier();  // every wave is past its last z-plane read and parameter read
    auto part = [&](int w, int tile, int c) -> f4& {
      const int i = (w * 16 + tile) * 32 + c;  // 16 tiles a round
      return i < kZSlots ? s_z[i] : s_prm[i - kZSlots];
    };
    const int col = lane & 31;
    f4 yo[kPairs][2];
    // this wave's partials of round h (p is uniform over the wave: one branch, no selects)
    auto write_parts = [&](int h, auto P) __attribute__((always_inline)) {
#pragma unroll
      for (int r = 8 * h; r < 8 * h + 8; ++r) {
        float xo[2][2];
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const float m0 = acc[jj][0][r], m1 = acc[jj][1][r], m2 = acc[jj][2][r], m3 = acc[jj][3][r];
          xo[jj][0] = (m0 + m1) + m2;
          xo[jj][1] = (m1 - m2) - m3;
        }
        f4 pv;
        if constexpr (decltype(P)::value == 0)
          pv = f4{xo[0][0] + xo[1][0], xo[0][1] + xo[1][1], xo[1][0], xo[1][1]};
        else
          pv = f4{xo[0][0], xo[0][1], -(xo[0][0] + xo[1][0]), -(xo[0][1] + xo[1][1])};
        part(wave, 8 * (r >> 2) + 4 * g8 + (r & 3) - 16 * h, col) = pv;
      }
    };
#pragma unroll
    for (int h = 0; h < kPairs; ++h) {
      if (p == 0)
        write_parts(h, std::integral_constant<int, 0>{});
      else
        write_parts(h, std::integral_constant<int, 1>{});
      lds_barrier();
      {
        const int tile = tid >> 5, c = tid & 31;
        f4 pz[4];
#pragma unroll
        for (int z = 0; z < 4; ++z) pz[z] = part(2 * z, tile, c) + part(2 * z + 1, tile, c);
        const f4 y0 = (pz[0] + pz[1]) + pz[2];
        const f4 y1 = (pz[1] - pz[2]) - pz[3];
        yo[h][0] = y0 * a.out_scale;
        yo[h][1] = y1 * a.out_scale;
        if (a.bias) {
          const float bc = s_bias[c];
          yo[h][0] = yo[h][0] + bc;
          yo[h][1] = yo[h][1] + bc;
        }
      }
      lds_barrier();
    }
    wino_epilogue_tail(a, yo, reinterpret_cast<float*>(s_z), tid, lane, wave, cur.b, cur.nt,
                       cur.bzi, cur.byi, cur.bxi);
    if (!more) break;
    // the next box: its bias, and its item's parameters once every thread has read the tile
    // and the partials out of the parameter table
    if (nnt != cur.nt && tid < 32) s_bias[tid] = a.bias ? a.bias[nnt * 32 + tid] : 0.f;
    v = vnext;
    lds_barrier();
    load_prm(tid, wino_box(a, v).b);
  }
  // the last (zero-line) DMA lands before the workgroup's LDS is released
  __builtin_amdgcn_s_waitcnt(0);
}

// U[cout][cin][xi] = sum_{a,b,e} G[xz][a] G[xy][b] G[xx][e] w[cout][a][b][e][cin] in float64,
// times `scale`, rounded to float32, split into fp16 halves.  Word layout:
// packed[(((nt * chunks + chunk) * 64 + xi) * 2 + part) * 64 + lane], lane = column
// (cout = nt * 32 + lane % 32) and k slot (cin = chunk channel 8 * (lane / 32) + q).
__global__ void pack_wino_weight_kernel(const float* __restrict__ w, uint4* __restrict__ out,
                                        int cout, int c1, int c2, int chunks0, int chunks,
                                        int ntn, float scale) {
  const double G[4][3] = {{1.0, 0.0, 0.0}, {0.5, 0.5, 0.5}, {0.5, -0.5, 0.5}, {0.0, 0.0, 1.0}};
  const int cin_total = c1 + c2;
  const int64_t total = (int64_t)ntn * chunks * 64 * 64;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(i & 63);
    int64_t rest = i >> 6;
    const int xi = (int)(rest % 64);
    rest /= 64;
    const int chunk = (int)(rest % chunks);
    const int nt = (int)(rest / chunks);
    const int xz = xi >> 4, xy = (xi >> 2) & 3, xx = xi & 3;
    const int n = nt * 32 + (lane & 31);
    h8 hv, lv;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int k = 8 * (lane >> 5) + q;
      int wc = -1;
      if (chunk < chunks0) {
        const int cc = chunk * kWChunk + k;
        if (cc < c1) wc = cc;
      } else {
        const int cc = (chunk - chunks0) * kWChunk + k;
        if (cc < c2) wc = c1 + cc;
      }
      float v = 0.f;
      if (n < cout && wc >= 0) {
        double u = 0.0;
        for (int az = 0; az < 3; ++az)
          for (int ay = 0; ay < 3; ++ay)
            for (int ax = 0; ax < 3; ++ax) {
              const double gw = G[xz][az] * G[xy][ay] * G[xx][ax];
              if (gw != 0.0)
                u += gw * (double)w[(((int64_t)n * 3 + az) * 3 + ay) * 3 * cin_total +
                                    (int64_t)ax * cin_total + wc];
            }
        v = (float)(u * (double)scale);
      }
      const _Float16 h = (_Float16)v;
      hv[q] = h;
      lv[q] = (_Float16)(v - (float)h);
    }
    const int64_t word = ((((int64_t)nt * chunks + chunk) * 64 + xi) * 2) * 64 + lane;
    out[word] = *reinterpret_cast<const uint4*>(&hv);
    out[word + 64] = *reinterpret_cast<const uint4*>(&lv);
  }
}

}  // namespace

// Compute units of the current device, rounded down to a multiple of the 8 XCDs (the
// persistent kernel's grid: one workgroup a CU).
static int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  hip_check(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= 64) dev = 0;
  if (cached[dev] == 0) {
    int n = 0;
    hip_check(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev),
              "hipDeviceGetAttribute");
    cached[dev] = n >= 8 ? n / 8 * 8 : 8;
  }
  return cached[dev];
}

// NNX_WINO_PERSISTENT=0 keeps every Winograd layer on the one-box-a-workgroup kernel (read
// at each launch, for comparisons).
static bool wino_persistent_enabled() {
  const char* e = std::getenv("NNX_WINO_PERSISTENT");
  return !(e && e[0] == '0');
}

// Layers outside this set take the direct split kernel (the route is chosen with it).
bool conv_wino_supported(const ConvGeom& g, int c1, int c2, int cout) {
  for (int i = 0; i < 3; ++i)
    if (g.k[i] != 3 || g.s[i] != 1) return false;
  return cout % 32 == 0 && c1 % kWChunk == 0 && c2 % kWChunk == 0 && c1 > 0 && c2 >= 0 &&
         c1 + c2 <= kMaxChannels;
}

int conv_wino_stats_tiles(const ConvGeom& g) {
  return (int)(ceil_div(g.out[0], 4) * ceil_div(g.out[1], 8) * ceil_div(g.out[2], 8));
}

float wino_weight_scale(float max_abs) {
  // |U| <= (1.5)^3 max |w|: the scale keeps every split high half below 2^15 (the bound in
  // float32, or in float64 where the float32 product would overflow)
  require(std::isfinite(max_abs) && max_abs >= 0.f, "weight magnitude must be finite");
  const float bound = 3.375f * max_abs;
  return split_weight_scale(std::isfinite(bound) ? (double)bound : 3.375 * (double)max_abs);
}

int64_t conv_wino_packed_bytes(int cout, int c1, int c2) {
  const int64_t chunks = ceil_div(c1, kWChunk) + ceil_div(c2, kWChunk);
  return ceil_div(cout, 32) * chunks * 64 * 2 * 64 * 16;
}

void conv_wino_pack_weight(const float* d_w, int cout, int c1, int c2, float scale,
                           void* d_packed, hipStream_t st) {
  require(d_w && d_packed, "Winograd packing pointers must not be null");
  require(cout >= 1 && c1 >= 1 && c2 >= 0, "invalid Winograd convolution channel counts");
  require(scale > 0.f && std::isfinite(scale), "weight scale must be positive");
  const int chunks0 = (int)ceil_div(c1, kWChunk);
  const int chunks = chunks0 + (int)ceil_div(c2, kWChunk);
  const int ntn = (int)ceil_div(cout, 32);
  const int64_t total = (int64_t)ntn * chunks * 64 * 64;
  const int blocks = (int)std::min<int64_t>(ceil_div(total, 256), 65536);
  hipLaunchKernelGGL(pack_wino_weight_kernel, dim3(blocks), dim3(256), 0, st, d_w,
                     reinterpret_cast<uint4*>(d_packed), cout, c1, c2, chunks0, chunks, ntn,
                     scale);
  launch_check("conv3d_winograd_pack_weight");
}

void conv3d_wino(const float* x1, int c1, const float* x2, int c2, const void* packed,
                 float scale, const float* bias, float* y, const ConvGeom& g, int cout,
                 hipStream_t st, float4* stats, const PendingNorm& n1, const PendingNorm& n2) {
  require(x1 && y && packed, "convolution pointers must not be null");
  require(c2 == 0 || x2, "invalid convolution inputs");
  require(conv_wino_supported(g, c1, c2, cout),
          "the Winograd convolution takes stride-1 3x3x3 layers with C_out % 32 == 0 and input "
          "channel counts that are multiples of 16, at most 1024 input channels in all");
  require(scale > 0.f && std::isfinite(scale), "weight scale must be positive");
  require(!(n1.params && n2.params) || n1.slope == n2.slope,
          "pending normalisations of one convolution must share the LeakyReLU slope");
  require(reinterpret_cast<uintptr_t>(y) % 16 == 0 && reinterpret_cast<uintptr_t>(x1) % 16 == 0 &&
              reinterpret_cast<uintptr_t>(x2) % 16 == 0,
          "Winograd convolution tensors must be 16-byte aligned");
  WinoArgs a{};
  a.x0 = x1;
  a.x1 = x2;
  a.c0 = c1;
  a.c1 = c2;
  a.chunks0 = c1 / kWChunk;
  a.chunks = a.chunks0 + c2 / kWChunk;
  a.u = reinterpret_cast<const uint4*>(packed);
  a.bias = bias;
  a.y = y;
  a.D = g.in[0];
  a.H = g.in[1];
  a.W = g.in[2];
  a.cout = cout;
  a.ntn = cout / 32;
  a.nbz = (int)ceil_div(g.out[0], 4);
  a.nby = (int)ceil_div(g.out[1], 8);
  a.nbx = (int)ceil_div(g.out[2], 8);
  const int64_t nwg = (int64_t)g.batch * a.nbz * a.nby * a.nbx * a.ntn;
  require(nwg < (1LL << 31), "convolution grid too large");
  a.nwg = (int)nwg;
  a.out_scale = 1.0f / scale;
  a.stats = stats;
  a.nrm0 = n1.params;
  a.nrm1 = n2.params;
  a.act0 = n1.act ? 1 : 0;
  a.act1 = n2.act ? 1 : 0;
  a.slope = n1.params ? n1.slope : n2.slope;
  const double out_vox = (double)g.batch * g.out[0] * g.out[1] * g.out[2];
  const double flops = 2.0 * (c1 + c2) * cout * 27.0 * out_vox;
  const double bytes = 4.0 * ((double)g.batch * g.in[0] * g.in[1] * g.in[2] * (c1 + c2) +
                              out_vox * cout);
  ProfScope prof("conv3d_wino", flops, bytes, st);
  const int cus = device_cus();
  if (a.chunks % 2 == 0 && wino_persistent_enabled() && a.nwg >= 4 * cus) {
    a.nbox = a.nwg / a.ntn;
    a.nvirt = a.nwg;
    hipLaunchKernelGGL(wino_x3p_kernel, dim3(cus), dim3(kWThreads), 0, st, a);
  } else {
    hipLaunchKernelGGL(wino_x3_kernel, dim3(a.nwg), dim3(kWThreads), 0, st, a);
  }
  launch_check("conv3d_winograd");
}

}  // namespace nnx
