// Internal helpers shared by the HIP sources of libnnunet_hip.so: error plumbing,
// launch checks and small device utilities.  Nothing here crosses the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>

#include "../../include/nnx.h"

namespace nnx {

// Thrown inside the library, converted to a status code + message at the ABI boundary.
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& msg) : std::runtime_error(msg), code(c) {}
};

void set_last_error(const std::string& msg);

[[noreturn]] inline void fail(int code, const std::string& msg) { throw Error(code, msg); }

inline void require(bool ok, const std::string& msg) {
  if (!ok) fail(NNX_ERR_INVALID, msg);
}

inline void hip_check(hipError_t err, const char* what) {
  if (err != hipSuccess) {
    fail(err == hipErrorOutOfMemory ? NNX_ERR_NOMEM : NNX_ERR_HIP,
         std::string(what) + ": " + hipGetErrorString(err));
  }
}

// Check the launch itself (bad configuration etc.).
inline void launch_check(const char* name) { hip_check(hipGetLastError(), name); }

// Wrap an ABI body: convert exceptions into status codes.
template <class F>
int guarded(F&& body) {
  try {
    body();
    return NNX_OK;
  } catch (const Error& e) {
    set_last_error(e.what());
    return e.code;
  } catch (const std::bad_alloc&) {
    set_last_error("host allocation failed");
    return NNX_ERR_NOMEM;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return NNX_ERR_STATE;
  }
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Physical workgroup ids are dealt round-robin to the 8 XCDs of an MI355X.  This maps a
// physical id to a logical id so that each XCD receives one contiguous range of logical
// ids (neighbouring tiles share halos and weights through that XCD's L2).  Bijective on
// [0, n) for any n.
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  constexpr int kXcd = 8;
  const int q = n / kXcd, r = n % kXcd;
  const int xcd = bid % kXcd, idx = bid / kXcd;
  return xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
}

}  // namespace nnx

// Optional per-launch timing with HIP events recorded on the launch stream.  When
// profiling is off (the default) a ProfScope costs one branch.
namespace nnx {

bool prof_enabled();
void prof_start(const char* name, double flops, double bytes, hipStream_t st);
void prof_stop(hipStream_t st);

struct ProfScope {
  hipStream_t st;
  bool on;
  ProfScope(const char* name, double flops, double bytes, hipStream_t s) : st(s), on(prof_enabled()) {
    if (on) prof_start(name, flops, bytes, st);
  }
  ~ProfScope() {
    if (on) prof_stop(st);
  }
};

}  // namespace nnx

// Kernel launcher entry points shared between the kernel files and the runtime.
namespace nnx {

struct ConvGeom {
  int batch;
  int in[3];
  int out[3];
  int k[3];
  int s[3];
  int p[3];
};

ConvGeom make_conv_geom(int batch, const int* in_size, const int* ksize, const int* stride);

// Packed weight helpers (device layout described in nnx_conv.hip).
int64_t conv_packed_floats(int cout, const int* ksize, int c1, int c2);
void conv_pack_weight(const float* d_w, int cout, const int* ksize, int c1, int c2,
                      float* d_packed, hipStream_t st);
// A convolution input may carry a pending InstanceNorm (+ LeakyReLU): its consumer applies
// r = fma(x - mean, scale, beta), then max(slope * r, r) when `act`, to every in-volume
// element it loads, with the same float32 operations as instnorm_apply_params (the zero
// padding stays zero).  `params` = (mean, scale, beta, 0) per (batch item, channel).
struct PendingNorm {
  const float4* params = nullptr;  // null: the tensor is already final
  bool act = false;
  float slope = 0.f;
};

// When `stats` is given, the epilogue also writes InstanceNorm partials
// stats[(b * tiles + tile) * cout + c] = (tile mean, tile M2, tile voxel count, 0) of
// (conv + bias); `tiles` = conv_stats_tiles(...) per batch item.
void conv3d_igemm(const float* x1, int c1, const float* x2, int c2, const float* packed,
                  const float* bias, float* y, const ConvGeom& g, int cout, hipStream_t st,
                  float4* stats = nullptr, const PendingNorm& n1 = {},
                  const PendingNorm& n2 = {});
int conv_stats_tiles(const ConvGeom& g, int cout, int c1, int c2);

// Split-fp16 implicit GEMM: float32 operands split into fp16 high/low halves, three MFMA
// products per term, float32 accumulation.  `scale` (a power of two from
// split_weight_scale) multiplies the weights before the split and is undone in the
// epilogue.  Activations must stay below the fp16 maximum (65504) in magnitude.
float split_weight_scale(double max_abs);
int64_t conv_x3_packed_bytes(int cout, const int* ksize, int c1, int c2);
// Operand arithmetic of the split kernels: kArithSplit3 = fp16 hi/lo halves, three
// products (float32 class); kArithBf16 = bf16 operands (round to nearest even), one
// product.  Both accumulate in float32; the packed layout and size are the same.
constexpr int kArithSplit3 = 0;
constexpr int kArithBf16 = 1;
void conv_x3_pack_weight(const float* d_w, int cout, const int* ksize, int c1, int c2,
                         float scale, void* d_packed, hipStream_t st, int arith = kArithSplit3);
void conv3d_x3(const float* x1, int c1, const float* x2, int c2, const void* packed,
               float scale, const float* bias, float* y, const ConvGeom& g, int cout,
               hipStream_t st, float4* stats = nullptr, const PendingNorm& n1 = {},
               const PendingNorm& n2 = {}, int arith = kArithSplit3);
int conv_x3_stats_tiles(const ConvGeom& g, int cout);

// Winograd F(2x2x2, 3x3x3) convolution with split-fp16 products (nnx_wino.hip): stride-1
// 3x3x3 layers with C_out % 32 == 0 and input channel counts that are multiples of 16.
// Weights are transformed (U = G w G^T per input/output channel pair), multiplied by
// `scale` (wino_weight_scale) and split at packing; stats as conv3d_x3 with tiles =
// conv_wino_stats_tiles (4 x 8 x 8 output boxes).
bool conv_wino_supported(const ConvGeom& g, int c1, int c2, int cout);
int conv_wino_stats_tiles(const ConvGeom& g);
float wino_weight_scale(float max_abs);
int64_t conv_wino_packed_bytes(int cout, int c1, int c2);
void conv_wino_pack_weight(const float* d_w, int cout, int c1, int c2, float scale,
                           void* d_packed, hipStream_t st);
void conv3d_wino(const float* x1, int c1, const float* x2, int c2, const void* packed,
                 float scale, const float* bias, float* y, const ConvGeom& g, int cout,
                 hipStream_t st, float4* stats = nullptr, const PendingNorm& n1 = {},
                 const PendingNorm& n2 = {});
// Whether the split kernel handles this kernel size / stride (tap count and halo size).
bool conv_x3_supported(const int* ksize, const int* stride, int cout);
// With `stats`: per-block InstanceNorm partials, conv_direct_stats_tiles(size) per item.
// wscale 0: float32 fma products; wscale > 0 (split_weight_scale of max |w|): split-fp16
// products on MFMA, each tile's input scaled by a power of two from its own max |x|; with
// split products the input may have 1, 2 or 4 channels (NDHWC, weights (C_out, 3, 3, 3, cin)).
void conv3d_direct_cin1(const float* x, const float* w, const float* bias, float* y, int batch,
                        const int* size, int cout, hipStream_t st, float4* stats = nullptr,
                        float wscale = 0.f, int cin = 1);
int conv_direct_stats_tiles(const int* size, bool split = false);

int64_t tconv_packed_floats(int cout, const int* ksize, int cin);
void tconv_pack_weight(const float* d_w, int cout, const int* ksize, int cin, float* d_packed,
                       hipStream_t st);
void tconv3d_gemm(const float* x, int cin, const float* packed, const float* bias, float* y,
                  int batch, const int* in_size, int cout, const int* ksize, hipStream_t st);
// Split-fp16 transposed convolution (stride == kernel), weights scaled like conv3d_x3.  With
// `norm` the input's pending InstanceNorm (+ LeakyReLU) is applied as its rows are staged
// (the same float32 operations as the apply pass); see tconv_norm_on_load.
int64_t tconv_x3_packed_bytes(int cout, const int* ksize, int cin);
void tconv_x3_pack_weight(const float* d_w, int cout, const int* ksize, int cin, float scale,
                          void* d_packed, hipStream_t st, int arith = kArithSplit3);
void tconv3d_x3(const float* x, int cin, const void* packed, float scale, const float* bias,
                float* y, int batch, const int* in_size, int cout, const int* ksize,
                hipStream_t st, int arith = kArithSplit3, const PendingNorm& norm = {});
// Whether tconv3d_x3 can take a pending norm for an input of this spatial size (its row
// tiles must not straddle batch items).
bool tconv_norm_on_load(const int* in_size);
// Class-logit restoration: half-pixel trilinear (edge-clamped, float64) resampling of
// channels-last logits (src[0], src[1], src[2], classes) to dst, then first-maximum argmax
// into uint16 labels (dst[0], dst[1], dst[2]).  `half`: float16 logits, values rounded to
// float16 before the comparison.
void restore_labels(const void* logits, bool half, int classes, const int* src, const int* dst,
                    uint16_t* labels, hipStream_t st);
// Raw-case preprocessing (nnx_preprocess.hip).
void nonzero_bbox(const float* x, int channels, const int64_t* size, int* bbox, hipStream_t st);
void crop_normalize(const float* x, int channels, const int64_t* size, const int* transpose,
                    const int64_t* start, const int64_t* out_size, const int* schemes,
                    const float* norm, float* out, hipStream_t st);
void crop_normalize_masked(const float* x, int channels, const int64_t* size,
                           const int* transpose, const int64_t* start, const int64_t* out_size,
                           const int* schemes, const float* norm, const uint8_t* mask,
                           const int64_t* mask_start, const int64_t* mask_extent, float* out,
                           hipStream_t st);
// Filled nonzero mask of the raw box (start, extent): returns the number of sweep rounds.
int nonzero_mask_filled(const float* x, int channels, const int64_t* size, const int64_t* start,
                        const int64_t* extent, uint8_t* mask, void* work, hipStream_t st);
size_t zscore_stats_workspace();
void box_minmax(const float* x, int channels, const int64_t* size, int channel,
                const int64_t* start, const int64_t* extent, float* minmax, void* work,
                hipStream_t st);
void zscore_stats(const float* x, int channels, const int64_t* size, int channel,
                  const int64_t* start, const int64_t* extent, const uint8_t* mask, float* stats,
                  void* work, hipStream_t st);
size_t resample_spline_workspace(const int64_t* size, const int64_t* new_size, int separate_axis);
void resample_spline(const float* x, int channels, const int64_t* size, const int64_t* new_size,
                     int order, int separate_axis, int order_z, void* work, size_t work_bytes,
                     float* out, hipStream_t st, bool round_half = false);
// Class-logit restoration along a spline plan: each class of channels-last logits
// (src, classes) resampled like resample_spline (rounded to float16 when `half`), then the
// first-maximum argmax into uint16 labels (dst); one class at a time through `work`.
// Torch-grid resampling (nnx_torchgrid.hip): one pass, strided (channel, axis 0, 1, 2),
// float32 or float16 (`half`) input, float32 output; torch_resize_argmax resamples every
// class of a voxel and writes the first-maximum label (contiguous uint16 labels).
void torch_resize(const void* in, bool half, int channels, const int* in_size,
                  const int64_t* in_strides, float* out, const int* out_size,
                  const int64_t* out_strides, int mode, hipStream_t st);
void torch_resize_argmax(const void* in, bool half, int classes, const int* in_size,
                         const int64_t* in_strides, const int* out_size, int mode,
                         uint16_t* labels, hipStream_t st);
size_t restore_labels_spline_workspace(const int* src, const int* dst, int separate_axis);
void restore_labels_spline(const void* logits, bool half, int classes, const int* src,
                           const int* dst, int order, int separate_axis, void* work,
                           size_t work_bytes, uint16_t* labels, hipStream_t st);
// `item_voxels` = voxels per batch item (to index the pending norm's parameters).
void conv1x1(const float* x, int cin, const float* w, const float* bias, float* y,
             int64_t voxels, int cout, hipStream_t st, const PendingNorm& nx = {},
             int64_t item_voxels = 0);

size_t instnorm_workspace_bytes(int batch, int64_t spatial, int channels);
size_t instnorm_noalloc_max_bytes();
void instnorm_lrelu_noalloc(const float* x, float* y, int batch, int64_t spatial, int channels,
                            const float* input_bias, const float* gamma, const float* beta,
                            float eps, bool act, float slope, const float* residual,
                            hipStream_t st);
void instnorm_lrelu(const float* x, float* y, int batch, int64_t spatial, int channels,
                    const float* input_bias, const float* gamma, const float* beta, float eps,
                    bool act, float slope, const float* residual, void* ws, size_t ws_bytes,
                    hipStream_t st);
// InstanceNorm parameters only: params[b * channels + c] = (mean, gamma*rsqrt(var+eps), beta,
// 0) of (x + input_bias); written to `params`, or into the workspace when params is null.
void instnorm_params(const float* x, int batch, int64_t spatial, int channels,
                     const float* input_bias, const float* gamma, const float* beta, float eps,
                     void* ws, size_t ws_bytes, float4* params, hipStream_t st);
// The same parameters from per-tile partials (mean, M2, n, 0) written by a convolution
// epilogue.  The partials are consumed: the merge overwrites them.
void instnorm_merge_partials(float4* partials, int nparts, int batch, int64_t spatial,
                             int channels, const float* gamma, const float* beta, float eps,
                             float4* params, hipStream_t st);
// y = LeakyReLU?(fma(x + input_bias - mean, scale, beta) (+ residual)), elementwise.
void instnorm_apply_params(const float* x, float* y, int batch, int64_t spatial, int channels,
                           const float4* params, const float* input_bias, bool act, float slope,
                           const float* residual, hipStream_t st);
void avgpool3d(const float* x, float* y, int batch, const int* in_size, int channels,
               const int* kernel, hipStream_t st);

// Centred crop / zero pad of an NDHWC tensor to out_size (the decoder's _match_spatial).
void match_spatial(const float* x, const int* in_size, float* y, const int* out_size, int batch,
                   int channels, hipStream_t st);

void count_nonfinite(const float* x, int64_t n, unsigned int* count, hipStream_t st);

void sw_gather_flip(const float* vol, int channels, const int64_t* size, const int* pad_before,
                    const int* offset, const int* patch, const int* flips, int nviews,
                    float* out, hipStream_t st);
void sw_accumulate(const float* pred, int nviews, const int* flips, int k, const int* patch,
                   const void* gaussian, const int* offset, const int64_t* padded, int accum,
                   void* acc, void* norm, hipStream_t st);
void sw_fold_add(const void* acc, const void* norm, int k, const int64_t* padded,
                 const int* crop_lo, const int64_t* crop_size, int accum, bool first,
                 void* total, hipStream_t st);
void sw_fold_finalize(const void* total, int k, int64_t voxels, int nfolds, int accum,
                      void* logits, uint16_t* labels, unsigned int* invalid, hipStream_t st);
void fill_zero(void* ptr, size_t bytes, hipStream_t st);

}  // namespace nnx
