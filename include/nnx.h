/*
 * nnx.h — C ABI of libnnunet_hip.so, the MI355X (gfx950) nnU-Net v2 inference path.
 *
 * Every entry point takes plain pointers, sizes and a hipStream_t (passed as void*),
 * returns an int status (NNX_OK = 0, negative = error class) and never lets a C++
 * exception cross the boundary.  nnx_last_error() returns the thread-local message of
 * the last failure.  Device pointers are caller-owned unless stated otherwise; the
 * library owns model weights and the activation/accumulator workspace it allocates at
 * create/load time or on the first call at a new shape (never inside the tile loop).
 *
 * Layouts follow the reference (MedMLX/nnunet-mlx): activations are channels-last
 * NDHWC float32 (src/nnunet_mlx/model/network.py:1-7); convolution weights are
 * (C_out, kD, kH, kW, C_in) (src/nnunet_mlx/storage/weights.py:32-45); sliding-window
 * volumes are channels-first (C, Z, Y, X) (src/nnunet_mlx/prediction/sliding_window.py:131).
 */
#ifndef NNX_H
#define NNX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------------- */
#define NNX_OK 0
#define NNX_ERR_INVALID (-1)   /* contract violation: shapes, arguments (ContractError) */
#define NNX_ERR_HIP (-2)       /* HIP runtime error */
#define NNX_ERR_NONFINITE (-3) /* non-finite logits (ContractError) */
#define NNX_ERR_STATE (-4)     /* missing/duplicate parameters, wrong call order */
#define NNX_ERR_NOMEM (-5)     /* device allocation failed */

/* Thread-local message of the last failed call on this thread.
 * Replaces: ContractError messages, src/nnunet_mlx/errors.py:4. */
const char* nnx_last_error(void);

/* Library version string and the gfx target the code objects were built for. */
const char* nnx_version(void);

/* ---- network seam --------------------------------------------------------------
 * Replaces the InferenceModel protocol (src/nnunet_mlx/model/types.py:17-32) built by
 * build_model_from_plans (src/nnunet_mlx/model/factory.py:17-65) from
 * PlainConvUNetSpec / ResidualEncoderUNetSpec (src/nnunet_mlx/model/topology.py:132,257).
 */
#define NNX_ARCH_PLAIN 0
#define NNX_ARCH_RESIDUAL 1
#define NNX_PRECISION_FP32 0
/* Float32 semantics (float32 inputs, weights, accumulation and outputs) with the 3-D
 * convolutions computed as three fp16 MFMA products of split operands (x = hi + lo), see
 * nnx_conv3d_split.  A first convolution with 1, 2 or 4 input channels uses split products
 * too, with a per-tile power-of-two scale of the raw input (nnx_conv3d_direct_small_cin_split);
 * other first convolutions keep float32 products.  Meets the float32 logits tolerance;
 * hidden activations must stay below 65504 in magnitude at layers on the direct split kernels
 * and below 8188 at the Winograd layers (the input transform sums up to 8 of them before the
 * split).  They are InstanceNorm outputs, so with ordinary affine parameters they do; a
 * checkpoint whose activations exceed the range makes the forward fail with a ContractError
 * that names the layer (nnx_set_layer_checks), never a silent result. */
#define NNX_PRECISION_FP32_SPLIT 1
/* bf16 operands with float32 accumulation (the pancreas config's bf16): the 3-D
 * convolutions after the first one and the transposed convolutions round their weights
 * and input activations to bf16 (nearest even) and multiply on bf16 MFMA, accumulating in
 * float32; InstanceNorm statistics, the first convolution, 1x1x1 convolutions and the
 * activations between layers stay float32.  On random-init networks the logits land at
 * relative-L2 1.0e-2 to 2.3e-2 of the float32 logits, the distance the same bf16 rounding
 * reaches when emulated on the CPU; relative-L2 1e-2 is not met in general. */
#define NNX_PRECISION_BF16 2
/* bf16 below full resolution: as NNX_PRECISION_BF16 for every layer whose output is below
 * the network's full resolution (encoder stages >= 1, decoder stages and transposed
 * convolutions that end below full resolution), NNX_PRECISION_FP32_SPLIT for the
 * full-resolution encoder stage (the stem included), the last decoder stage and the
 * transposed convolution into it.  On the pancreas ResEnc-L (128 x 160 x 160) two thirds of
 * the convolution FLOPs run in bf16 and the logits land at relative-L2 7.6e-3 of the
 * float32 logits (all-bf16: 1.2e-2). */
#define NNX_PRECISION_BF16_MIXED 3

typedef struct nnx_spec {
  int arch;              /* NNX_ARCH_PLAIN or NNX_ARCH_RESIDUAL */
  int spatial_dims;      /* 3 (2-D networks are rejected) */
  int input_channels;     /* 1..1024 */
  int num_classes;        /* 1..1024 */
  int n_stages;           /* 2..16 */
  const int* features;      /* n_stages, each 1..1024 (the InstanceNorm's channel limit) */
  const int* kernel_sizes;  /* n_stages * 3, odd, 1..15 */
  const int* strides;       /* n_stages * 3, 1..16 */
  const int* encoder_convs; /* n_stages: convs per stage (plain) or blocks per stage (residual),
                               1..64 */
  const int* decoder_convs; /* n_stages - 1, 1..64 */
  int conv_bias;
  int norm_affine;
  float norm_eps;
  float leaky_slope;
  int stem_channels; /* residual only; 0 means features[0]; at most 1024 */
  const int* bottleneck_channels; /* residual only: n_stages entries (1..1024) for
                                     BottleneckD, or NULL for BasicBlockD */
  int precision;     /* NNX_PRECISION_FP32, _FP32_SPLIT, _BF16 or _BF16_MIXED */
} nnx_spec;

typedef struct nnx_model nnx_model;

/* Build the layer graph of a network; no weights yet.  A field outside the ranges above
 * returns NNX_ERR_INVALID.
 * Replaces PlainConvUNet/ResidualEncoderUNet __init__ (src/nnunet_mlx/model/network.py:422-451,664-699). */
int nnx_model_create(const nnx_spec* spec, nnx_model** out);

/* Number of parameters the graph expects, and the name/shape of parameter i (reference
 * key names, e.g. "enc0.block1.conv.weight", "up2.bias", "seg4.weight"). */
int nnx_model_param_count(const nnx_model* model, int* count);
int nnx_model_param_info(const nnx_model* model, int index, const char** name, int* ndim,
                         int64_t* shape /* 5 entries */);

/* Load one float32 host parameter by reference key name and MLX layout.
 * Replaces load_inference_checkpoint's strict safetensors load
 * (src/nnunet_mlx/storage/checkpoint.py:130-165,232-237). */
int nnx_model_load_param(nnx_model* model, const char* name, const float* host,
                         const int64_t* shape, int ndim);

/* Check that every parameter was loaded exactly once and is finite, repack weights into
 * the MFMA fragment layouts and upload them.  Required before nnx_forward.  A call that
 * fails for missing parameters can be repeated after loading them; one that fails later
 * (a device error while uploading or packing) leaves the model unusable: every later call
 * fails with NNX_ERR_INVALID, and the model is destroyed and rebuilt. */
int nnx_model_finalize(nnx_model* model);

/* Let `model` use the activation workspace of `owner` (fold ensembles keep every fold's
 * weights resident but run one fold at a time).  Calls on models sharing a workspace
 * must be serialised by the caller. */
int nnx_model_share_workspace(nnx_model* model, nnx_model* owner);

/* Forward n channels-last tiles (n, D, H, W, C_in) -> (n, D, H, W, num_classes) float32.
 * Replaces PlainConvUNet.__call__ / ResidualEncoderUNet.__call__
 * (src/nnunet_mlx/model/network.py:453-464,701-728). */
int nnx_forward(nnx_model* model, const float* d_in, float* d_out, int n, const int* spatial,
                void* stream);

void nnx_model_destroy(nnx_model* model);

/* ---- sliding-window seam --------------------------------------------------------
 * Replaces _accumulate_logits + finalizers + fold averaging
 * (src/nnunet_mlx/prediction/sliding_window.py:158-460, src/nnunet_mlx/prediction/inference.py:93-149).
 * Tile offsets, mirror order and the Gaussian map are computed by the host layer
 * (bit-exact with the reference's numpy arithmetic) and passed in.
 */
#define NNX_ACCUM_F32 0
#define NNX_ACCUM_NNUNET_F16 1

typedef struct nnx_sw_config {
  int channels;             /* C_in of the volume */
  int num_classes;          /* K */
  int64_t size[3];          /* unpadded volume size (Z, Y, X) */
  int pad_before[3];        /* minimum zero padding before each axis (_pad_minimum) */
  int64_t padded[3];        /* padded size = size + pad */
  int patch[3];
  int ntiles;
  const int* tile_offsets;  /* host, ntiles * 3, padded coordinates, itertools.product order */
  int nviews;               /* 1 + number of mirrored views */
  const int* view_flips;    /* host, nviews bitmasks: 1 = axis 0 (z), 2 = axis 1 (y), 4 = axis 2 (x) */
  int accumulation;         /* NNX_ACCUM_F32 or NNX_ACCUM_NNUNET_F16 */
  const void* d_gaussian;   /* device, patch voxels, float32 (F32) or float16 (NNUNET_F16) */
  int tiles_per_batch;      /* tiles sharing one forward batch (views * tiles_per_batch) */
} nnx_sw_config;

/* Forward callback for custom networks: d_in (n, *patch, C) -> d_out (n, *patch, K). */
typedef int (*nnx_forward_fn)(void* user, const float* d_in, float* d_out, int n,
                              const int* spatial, void* stream);

/* Fold-averaged sliding-window prediction on one GPU.  d_volume is (C, Z, Y, X) float32.
 * Outputs (either may be NULL): d_logits cropped channels-last (Z, Y, X, K) in the
 * accumulation dtype (float32 or float16), equal to predict_device_logits /
 * average_fold_device_logits; d_labels cropped (Z, Y, X) uint16 argmax with
 * earliest-channel ties (predict_labels / normalized_labels).  Returns
 * NNX_ERR_NONFINITE when any cropped logit is non-finite. */
int nnx_sw_predict(nnx_model* const* folds, int nfolds, const nnx_sw_config* config,
                   const float* d_volume, void* d_logits, uint16_t* d_labels, void* stream);

/* Same with caller-supplied forward callbacks (one per fold). */
int nnx_sw_predict_custom(nnx_forward_fn const* forwards, void* const* users, int nfolds,
                          const nnx_sw_config* config, const float* d_volume, void* d_logits,
                          uint16_t* d_labels, void* stream);

/* Release the sliding-window accumulators cached by the library. */
void nnx_sw_release(void);

/* ---- kernel families (device pointers, caller-owned) ----------------------------- */

/* Layer checks on (1) or off (0) for every later forward of this process: after each
 * convolution, transposed convolution and head the stream is synchronised and the layer's
 * output scanned, and the first layer with non-finite values fails the forward with
 * NNX_ERR_NONFINITE and an error naming its parameter (NNX_CHECK_LAYERS=1 in the environment
 * turns them on for the whole process).  The host uses them to name the layer after a
 * forward has produced non-finite logits; they serialise the forward.
 * Replaces nothing in the reference, whose float32 path has no operand range: it names the
 * layer where the split-fp16 precisions meet theirs (its inputs beyond 65504, or beyond
 * 8188 at a Winograd layer, whose input transform adds up to 8 of them). */
int nnx_set_layer_checks(int enable);

/* Count non-finite float32 values; *d_count (device uint32) is overwritten.
 * Replaces the finite checks of _validate_request (src/nnunet_mlx/prediction/sliding_window.py:470-477). */
int nnx_count_nonfinite(const float* d_x, int64_t n, unsigned int* d_count, void* stream);

/* Fused InstanceNorm (+ input bias, + optional residual add) + optional LeakyReLU over the
 * spatial axes of a (B, S, C) float32 tensor; y may alias x.  y = max(slope*r, r) with
 * r = fma(x + b - mean, gamma*rsqrt(var+eps), beta) (+ residual when given, before the
 * activation).  Replaces instance_norm (src/nnunet_mlx/kernels/metal_native_norm.py:92-168)
 * and the residual add + leaky_relu of ResidualBlock (src/nnunet_mlx/model/network.py:511-516). */
size_t nnx_instnorm_workspace_bytes(int batch, int64_t spatial, int channels);
int nnx_instnorm_lrelu(const float* d_x, float* d_y, int batch, int64_t spatial, int channels,
                       const float* d_input_bias, const float* d_gamma, const float* d_beta,
                       float eps, int apply_act, float slope, const float* d_residual,
                       void* d_workspace, size_t workspace_bytes, void* stream);

/* nnx_instnorm_lrelu without a workspace and without any allocation: the partials and
 * parameters live in a file-scope device array of nnx_instnorm_noalloc_max_bytes() bytes
 * (16 MiB; each GPU keeps its own copy until the process ends).  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Sizes whose
 * nnx_instnorm_workspace_bytes() exceeds the scratch return NNX_ERR_INVALID.  Calls that
 * overlap on one GPU share the scratch and race; the caller serialises them. */
size_t nnx_instnorm_noalloc_max_bytes(void);
int nnx_instnorm_lrelu_noalloc(const float* d_x, float* d_y, int batch, int64_t spatial,
                               int channels, const float* d_input_bias, const float* d_gamma,
                               const float* d_beta, float eps, int apply_act, float slope,
                               const float* d_residual, void* stream);

/* Implicit-GEMM 3-D convolution on fp32 MFMA, NDHWC.  Two input pointers implement the
 * concat-free decoder convolution conv(concat(x1, x2)) (x2 may be NULL, c2 = 0).
 * Padding is k//2 per axis; the bias (may be NULL) is added to each output.
 * Replaces mx.conv3d via _unbiased_convolution (src/nnunet_mlx/model/network.py:240-269)
 * and the split concat convolution (src/nnunet_mlx/model/network.py:305-322). */
size_t nnx_conv3d_packed_floats(int cout, const int* ksize, int c1, int c2);
int nnx_conv3d_pack_weight(const float* d_weight /* (Cout,kD,kH,kW,c1+c2) */, int cout,
                           const int* ksize, int c1, int c2, float* d_packed, void* stream);
int nnx_conv3d_igemm(const float* d_x1, int c1, const float* d_x2, int c2,
                     const float* d_packed, const float* d_bias, float* d_y, int batch,
                     const int* in_size, int cout, const int* ksize, const int* stride,
                     void* stream);

/* The same convolution with float32 operands split into fp16 halves (hi = fp16(v),
 * lo = fp16(v - hi)) and summed as hi*hi + hi*lo + lo*hi on fp16 MFMA with float32
 * accumulation (relative error ~2^-21 per product).  Weights are multiplied by `scale`,
 * a power of two from nnx_split_weight_scale(max |w|), before the split (so their low
 * halves stay normal); outputs are multiplied by 1/scale (exact).  Packed size in bytes.
 * Replaces the same reference calls as nnx_conv3d_igemm. */
float nnx_split_weight_scale(float max_abs); /* 0 for a negative or non-finite argument */
size_t nnx_conv3d_split_packed_bytes(int cout, const int* ksize, int c1, int c2);
int nnx_conv3d_split_pack_weight(const float* d_weight /* (Cout,kD,kH,kW,c1+c2) */, int cout,
                                 const int* ksize, int c1, int c2, float scale, void* d_packed,
                                 void* stream);
int nnx_conv3d_split(const float* d_x1, int c1, const float* d_x2, int c2, const void* d_packed,
                     float scale, const float* d_bias, float* d_y, int batch, const int* in_size,
                     int cout, const int* ksize, const int* stride, void* stream);

/* The same convolution in Winograd form F(2x2x2, 3x3x3) for stride-1 3x3x3 layers with
 * C_out % 32 == 0 and c1, c2 multiples of 16: per 2x2x2 output tile the 4x4x4 input patch
 * and each 3x3x3 filter are transformed (additions, and halves for the filter: exact in
 * float32 / float64), the 64 transform positions are multiplied as split-fp16 products
 * (hi*hi + hi*lo + lo*hi, float32 accumulation) on fp16 MFMA, and the output transform
 * returns the tile; 64 products per 8 outputs instead of 216.  Filters are transformed in
 * float64, multiplied by `scale` (nnx_winograd_weight_scale(max |w|)) and split when
 * packed; outputs are multiplied by 1/scale (exact), + bias.  Replaces the same reference
 * calls as nnx_conv3d_igemm (mx.conv3d via _unbiased_convolution,
 * src/nnunet_mlx/model/network.py:240-269, and the split concat convolution,
 * src/nnunet_mlx/model/network.py:305-322). */
float nnx_winograd_weight_scale(float max_abs); /* 0 for a negative or non-finite argument */
size_t nnx_conv3d_winograd_packed_bytes(int cout, int c1, int c2);
int nnx_conv3d_winograd_pack_weight(const float* d_weight /* (Cout,3,3,3,c1+c2) */, int cout,
                                    int c1, int c2, float scale, void* d_packed, void* stream);
int nnx_conv3d_winograd(const float* d_x1, int c1, const float* d_x2, int c2,
                        const void* d_packed, float scale, const float* d_bias, float* d_y,
                        int batch, const int* in_size, int cout, void* stream);

/* One-input-channel 3x3x3 stride-1 pad-1 convolution, fma over taps in (kd,kh,kw) order.
 * Replaces single_channel_conv3d (src/nnunet_mlx/kernels/metal_single_channel_conv.py:32-97). */
int nnx_conv3d_direct_small_cin(const float* d_x, const float* d_weight /* (Cout,3,3,3,1) */,
                                const float* d_bias, float* d_y, int batch, const int* size,
                                int cout, void* stream);
/* The same convolution with split-fp16 products on MFMA for 1, 2 or 4 input channels (the
 * 27 * cin (tap, channel) products of 16 voxels as 16 x 32 fragments, hi*hi + hi*lo +
 * lo*hi, float32 accumulation): weights times `scale` (nnx_split_weight_scale of max |w|),
 * each 4 x 4 x 16 output tile's input (all channels) times one power of two from the tile's
 * own max |x|, products times the inverses (exact), + bias.  Replaces the same reference
 * call as nnx_conv3d_direct_small_cin in the fp32-split precision, and the first
 * Conv3d of two- and four-channel networks (mx.conv3d via _unbiased_convolution,
 * src/nnunet_mlx/model/network.py:240-269). */
int nnx_conv3d_direct_small_cin_split(const float* d_x, int cin /* 1, 2 or 4 */,
                                      const float* d_weight /* (Cout,3,3,3,cin) */, float scale,
                                      const float* d_bias, float* d_y, int batch,
                                      const int* size, int cout, void* stream);

/* Stride==kernel ConvTranspose3d as one MFMA GEMM whose epilogue writes the interleaved
 * output directly (no transpose pass), + bias.
 * Replaces NonOverlappingConvTranspose3d (src/nnunet_mlx/model/network.py:101-174). */
size_t nnx_tconv3d_packed_floats(int cout, const int* ksize, int cin);
int nnx_tconv3d_pack_weight(const float* d_weight /* (Cout,kD,kH,kW,Cin) */, int cout,
                            const int* ksize, int cin, float* d_packed, void* stream);
int nnx_tconv3d_gemm(const float* d_x, int cin, const float* d_packed, const float* d_bias,
                     float* d_y, int batch, const int* in_size, int cout, const int* ksize,
                     void* stream);

/* The same transposed convolution with split-fp16 products (hi*hi + hi*lo + lo*hi, float32
 * accumulation), weights multiplied by `scale` (nnx_split_weight_scale) before the split;
 * the tile is staged in LDS and written as contiguous channel runs.  Packed size in bytes.
 * Replaces the same reference call as nnx_tconv3d_gemm. */
size_t nnx_tconv3d_split_packed_bytes(int cout, const int* ksize, int cin);
int nnx_tconv3d_split_pack_weight(const float* d_weight /* (Cout,kD,kH,kW,Cin) */, int cout,
                                  const int* ksize, int cin, float scale, void* d_packed,
                                  void* stream);
int nnx_tconv3d_split(const float* d_x, int cin, const void* d_packed, float scale,
                      const float* d_bias, float* d_y, int batch, const int* in_size, int cout,
                      const int* ksize, void* stream);

/* The bf16 arithmetic (NNX_PRECISION_BF16) of the same two kernels: weights times `scale`
 * and input activations rounded to bf16 (nearest even), one bf16 MFMA product, float32
 * accumulation, outputs times 1/scale.  Packed sizes as nnx_conv3d_split_packed_bytes and
 * nnx_tconv3d_split_packed_bytes.  Replace the same reference calls as the split entries
 * (the reference has no bf16 path; these serve the bf16 config). */
int nnx_conv3d_bf16_pack_weight(const float* d_weight /* (Cout,kD,kH,kW,c1+c2) */, int cout,
                                const int* ksize, int c1, int c2, float scale, void* d_packed,
                                void* stream);
int nnx_conv3d_bf16(const float* d_x1, int c1, const float* d_x2, int c2, const void* d_packed,
                    float scale, const float* d_bias, float* d_y, int batch, const int* in_size,
                    int cout, const int* ksize, const int* stride, void* stream);
int nnx_tconv3d_bf16_pack_weight(const float* d_weight /* (Cout,kD,kH,kW,Cin) */, int cout,
                                 const int* ksize, int cin, float scale, void* d_packed,
                                 void* stream);
int nnx_tconv3d_bf16(const float* d_x, int cin, const void* d_packed, float scale,
                     const float* d_bias, float* d_y, int batch, const int* in_size, int cout,
                     const int* ksize, void* stream);

/* Restoration of class logits to the original grid: half-pixel trilinear resampling
 * (coordinates clamped to the source edges) of channels-last logits
 * (src_shape[0], src_shape[1], src_shape[2], classes) to dst_shape, evaluated in float64,
 * then the first-maximum argmax into uint16 labels (dst_shape). half != 0: the logits are
 * float16 and each interpolated value is rounded to float16 (nearest even) before the
 * comparison.  classes <= 65536.
 * Replaces the fused Metal restoration _launch / resample_device_logits_argmax
 * (src/nnunet_mlx/kernels/metal_restore.py:358-427, kernel :69-137). */
int nnx_restore_labels(const void* d_logits, int half, int classes, const int* src_shape,
                       const int* dst_shape, uint16_t* d_labels, void* stream);

/* Torch-grid resampling (the plans' resample_torch_fornnunet): one pass from in_size to
 * out_size over three spatial axes, mode 0 linear (align_corners=False half-pixel grid,
 * edge-clamped; the eight corner terms ((v * w0) * w1) * w2 summed in float64 in corner
 * order and rounded once to float32), 1 nearest (floor(i * S / T)) or 2 nearest-exact
 * (floor((i + 0.5) * S / T)), with float32 coordinates (scale = S / T in float32).
 * Input float32, or float16 when `half` (widened exactly); output float32.  Strides
 * (elements) are given for the channel and the three axes of input and output, so
 * channels-first images and channels-last logits are read and written in place.  A
 * separate-axis resampling is two calls: the planes across the axis with the plans' mode
 * (that axis kept at its size), then the whole volume with aniso_axis_mode.  At most 2^31
 * output elements.
 * Replaces torch_resize / resample_torch (src/nnunet_mlx/kernels/metal_torch_resample.py:
 * 136-215) for images and probabilities (is_seg false), as resample_probabilities_or_data
 * calls it (src/nnunet_mlx/data/resampling.py:127-145). */
int nnx_torch_resize(const void* d_in, int half, int channels, const int* in_size,
                     const int64_t* in_strides, float* d_out, const int* out_size,
                     const int64_t* out_strides, int mode, void* stream);

/* One Torch-grid pass of every class of (strided) logits followed by the first-maximum
 * argmax per output voxel, without a float intermediate: d_labels receives
 * out_size[0] x out_size[1] x out_size[2] contiguous uint16 labels (1..65536 classes,
 * at most 2^31 voxels).  The last pass of a Torch-plan class restoration.
 * Replaces resample_probabilities_or_data (Torch resampler) followed by the argmax of
 * the class-model export (src/nnunet_mlx/data/resampling.py:127-145,
 * src/nnunet_mlx/prediction/export.py:137-202). */
int nnx_torch_resize_argmax(const void* d_logits, int half, int classes, const int* in_size,
                            const int64_t* in_strides, const int* out_size, int mode,
                            uint16_t* d_labels, void* stream);

/* Restoration along the plans' spline resampler, for the cases the trilinear entry does not
 * take (separate-axis resampling with order_z 0, or order 3): each class of the
 * channels-last logits (src_shape, classes) is resampled to dst_shape as
 * nnx_resample_spline does (order 1 or 3, separate_axis -1 or 0..2), rounded once to
 * float32 — or to float16 when half != 0 (float16 logits) — and folded into a
 * first-maximum argmax (strict ">", ties keep the earliest class) written as uint16 labels.
 * One class at a time through a device workspace of
 * nnx_restore_labels_spline_workspace bytes (0 = invalid shapes).  Replaces the host
 * restoration resample_class_logits_argmax_parallel / separate_plane_argmax
 * (src/nnunet_mlx/prediction/restore.py:28-158) over resample_probabilities_or_data
 * (src/nnunet_mlx/data/resampling.py:87-172). */
size_t nnx_restore_labels_spline_workspace(const int* src_shape, const int* dst_shape,
                                           int separate_axis);
int nnx_restore_labels_spline(const void* d_logits, int half, int classes, const int* src_shape,
                              const int* dst_shape, int order, int separate_axis, void* d_work,
                              size_t work_bytes, uint16_t* d_labels, void* stream);

/* Raw-case preprocessing on the device (volumes are (C, X, Y, Z) float32, Z fastest, in
 * the array axis order of the raw image).
 *
 * nnx_nonzero_bbox: d_bbox[2a], d_bbox[2a + 1] = first and last index along axis a of a
 * voxel where any channel is nonzero (INT_MAX and -1 when there is none); the crop of
 * crop_to_nonzero without a mask (src/nnunet_mlx/data/preprocessing.py:166-214).
 *
 * nnx_crop_normalize: out (C, o0, o1, o2) with out axis k = input axis transpose[k] from
 * start[k] (out-axis order), each channel normalised by schemes[c]: NNX_NORM_NONE copies,
 * NNX_NORM_CT clips to [lower, upper] then (x - mean) / max(std, 1e-8) in float32, with
 * norm[4c..4c+3] = (mean, std, lower, upper); at most 16 channels.  Replaces the transpose
 * and crop of preprocess_raw_case and the CTNormalization / NoNormalization branches of
 * _normalize_channel (src/nnunet_mlx/data/preprocessing.py:100-128, 263-289).
 *
 * nnx_resample_spline: scikit-image resize(order, mode="edge", anti_aliasing=False) of each
 * channel to new_size (SciPy zoom in grid mode with edge extension, float64, clipped to the
 * input's [min, max]), order 1 or 3; with separate_axis in 0..2 the other two axes are
 * resized plane by plane (clipped per plane, float64) and separate_axis by half-pixel
 * nearest indices (order_z 0), rounded to float32 once.  The caller passes a device
 * workspace of nnx_resample_spline_workspace bytes.  Replaces resample_probabilities_or_data
 * for spline plans (src/nnunet_mlx/data/resampling.py:87-172, 268-306, 379-442, 476-501). */
#define NNX_NORM_NONE 0
#define NNX_NORM_CT 1
#define NNX_NORM_ZSCORE 2        /* (x - mean) / max(std, 1e-8), norm[4c..4c+1] = (mean, std) */
#define NNX_NORM_ZSCORE_MASKED 3 /* the same where the filled mask is set, else unchanged */
int nnx_nonzero_bbox(const float* d_data, int channels, const int64_t* size, int* d_bbox,
                     void* stream);
int nnx_crop_normalize(const float* d_data, int channels, const int64_t* size,
                       const int* transpose, const int64_t* start, const int64_t* out_size,
                       const int* schemes, const float* norm, float* d_out, void* stream);
/* Z-score normalisation (ZScoreNormalization of _normalize_channel,
 * src/nnunet_mlx/data/preprocessing.py:298-307, with the filled nonzero mask of
 * crop_to_nonzero, :166-214).
 *
 * nnx_nonzero_mask_filled: d_mask (extent[0], extent[1], extent[2]) uint8 over the raw box
 * at `start` = 1 where any channel is nonzero or the voxel lies in a background region
 * enclosed by it (6-connected, not connected to the box border: SciPy's
 * binary_fill_holes), else 0.  d_work: 256 bytes of device scratch.  Synchronises the
 * stream once per sweep round (not capturable); returns the round count (> 0) or a
 * negative error.
 *
 * nnx_zscore_stats: d_stats[0..1] = (mean, std) of channel `channel` over the raw box (only
 * mask voxels when d_mask is not null), accumulated in float64 and rounded to float32;
 * std about the float32 mean, biased (numpy's x.std()).  d_work: nnx_zscore_stats_workspace
 * bytes.
 *
 * nnx_crop_normalize_masked: nnx_crop_normalize with NNX_NORM_ZSCORE_MASKED channels, which
 * read d_mask over the raw box (mask_start, mask_extent) that contains the crop. */
int nnx_nonzero_mask_filled(const float* d_data, int channels, const int64_t* size,
                            const int64_t* start, const int64_t* extent, uint8_t* d_mask,
                            void* d_work, void* stream);
size_t nnx_zscore_stats_workspace(void);
int nnx_zscore_stats(const float* d_data, int channels, const int64_t* size, int channel,
                     const int64_t* start, const int64_t* extent, const uint8_t* d_mask,
                     float* d_stats, void* d_work, void* stream);
/* d_minmax[0..1] = (min, max) of channel `channel` over the raw box (start, extent);
 * d_work: nnx_zscore_stats_workspace bytes.  The extrema of RescaleTo01Normalization and the
 * range check of RGBTo01Normalization (src/nnunet_mlx/data/preprocessing.py:310-319); both
 * then normalise as NNX_NORM_ZSCORE with (mean, std) = (min, max(max - min, 1e-8)) and
 * (0, 255). */
int nnx_channel_minmax(const float* d_data, int channels, const int64_t* size, int channel,
                       const int64_t* start, const int64_t* extent, float* d_minmax,
                       void* d_work, void* stream);
int nnx_crop_normalize_masked(const float* d_data, int channels, const int64_t* size,
                              const int* transpose, const int64_t* start,
                              const int64_t* out_size, const int* schemes, const float* norm,
                              const uint8_t* d_mask, const int64_t* mask_start,
                              const int64_t* mask_extent, float* d_out, void* stream);
size_t nnx_resample_spline_workspace(const int64_t* size, const int64_t* new_size,
                                     int separate_axis);
int nnx_resample_spline(const float* d_data, int channels, const int64_t* size,
                        const int64_t* new_size, int order, int separate_axis, int order_z,
                        void* d_work, size_t work_bytes, float* d_out, void* stream);

/* 1x1x1 convolution with bias (segmentation head), NDHWC.
 * Replaces seg{n-1} (src/nnunet_mlx/model/network.py:804-808,875-876). */
int nnx_conv1x1(const float* d_x, int cin, const float* d_weight /* (Cout,1,1,1,Cin) */,
                const float* d_bias, float* d_y, int64_t voxels, int cout, void* stream);

/* Gather the tile at `offset` (padded coordinates) of a (C,Z,Y,X) volume, with virtual
 * zero padding, into nviews channels-last copies, view v flipped along view_flips[v].
 * Replaces volume[slices][None] + mx.flip/mx.contiguous
 * (src/nnunet_mlx/prediction/sliding_window.py:407-411,516-517). */
int nnx_sw_gather_flip(const float* d_volume, int channels, const int64_t* size,
                       const int* pad_before, const int* offset, const int* patch,
                       const int* view_flips, int nviews, float* d_out, void* stream);

/* Mirror-average the nviews outputs (flipped back, summed left to right in float32, / nviews)
 * and add them Gaussian-weighted into the padded (Z,Y,X,K) accumulator and (Z,Y,X)
 * normalizer.  F32: acc += p*g, norm += g.  NNUNET_F16: acc = f16(f32(acc) + p*f32(g)),
 * norm = f16(norm + g).
 * Replaces mirrored_prediction + the scatter-adds of _accumulate_logits
 * (src/nnunet_mlx/prediction/sliding_window.py:421-436,489-527). */
int nnx_sw_accumulate(const float* d_pred, int nviews, const int* view_flips, int num_classes,
                      const int* patch, const void* d_gaussian, const int* offset,
                      const int64_t* padded, int accumulation, void* d_acc, void* d_norm,
                      void* stream);

/* Normalise the cropped accumulator (f32(acc)/f32(norm), cast to the accumulation dtype)
 * into the fold total: total = normalized (first fold) or total + normalized.
 * Replaces predict_device_logits / add_fold_device_logits finalizers
 * (src/nnunet_mlx/prediction/sliding_window.py:242-249,285-302). */
int nnx_sw_fold_add(const void* d_acc, const void* d_norm, int num_classes, const int64_t* padded,
                    const int* crop_lo, const int64_t* crop_size, int accumulation, int first,
                    void* d_total, void* stream);

/* Divide the fold total by nfolds (float32, cast back; skipped for one fold), write the
 * optional logits and the argmax labels (earliest channel on ties; 65535 and a count in
 * *d_invalid for non-finite values).
 * Replaces average_fold_device_logits' division and normalized_labels' argmax
 * (src/nnunet_mlx/prediction/inference.py:140-149, src/nnunet_mlx/kernels/metal_normalized_labels.py:19-98). */
int nnx_sw_fold_finalize(const void* d_total, int num_classes, int64_t voxels, int nfolds,
                         int accumulation, void* d_logits, uint16_t* d_labels,
                         unsigned int* d_invalid, void* stream);

/* ---- kernel timing (no reference counterpart: measurement support) ----------------
 * Between nnx_profile_begin and nnx_profile_end every kernel launch of the library is
 * bracketed by HIP events on its own stream and attributed to a class (kernel name and
 * variant) with its algorithmic FLOPs and HBM bytes.  nnx_profile_end synchronises the
 * events; nnx_profile_read returns class `index` (0 <= index < *count). */
int nnx_profile_begin(void);
int nnx_profile_end(int* count);
int nnx_profile_read(int index, const char** name, int* launches, double* milliseconds,
                     double* flops, double* bytes);

/* AvgPool3d with kernel == stride on NDHWC (residual skip path).
 * Replaces _build_residual_skip's pool (src/nnunet_mlx/model/network.py:576-602). */
int nnx_avgpool3d(const float* d_x, float* d_y, int batch, const int* in_size, int channels,
                  const int* kernel, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* NNX_H */
