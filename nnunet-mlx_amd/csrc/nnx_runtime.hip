// Host runtime of libnnunet_hip.so: the network graph (PlainConvUNet and
// ResidualEncoderUNet with BasicBlockD/BottleneckD), parameter loading and repacking,
// the activation workspace, the forward pass and the GPU-resident sliding window, and
// every extern "C" entry point of include/nnx.h.
#include <atomic>
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "nnx_internal.h"

namespace nnx {

namespace {
thread_local std::string g_last_error;

struct ProfRecord {
  const char* name;
  hipEvent_t start, stop;
  double flops, bytes;
};

struct ProfTotal {
  std::string name;
  int launches = 0;
  double ms = 0, flops = 0, bytes = 0;
};

struct ProfState {
  std::mutex mu;
  bool on = false;
  std::vector<ProfRecord> records;
  std::vector<hipEvent_t> pool;
  std::vector<ProfTotal> totals;
};

ProfState& prof_state() {
  static ProfState* p = new ProfState();  // lives until process exit
  return *p;
}

hipEvent_t take_event(ProfState& p) {
  if (!p.pool.empty()) {
    hipEvent_t e = p.pool.back();
    p.pool.pop_back();
    return e;
  }
  hipEvent_t e;
  hip_check(hipEventCreate(&e), "hipEventCreate");
  return e;
}
}  // namespace

void set_last_error(const std::string& msg) { g_last_error = msg; }

bool prof_enabled() { return prof_state().on; }

void prof_start(const char* name, double flops, double bytes, hipStream_t st) {
  ProfState& p = prof_state();
  std::lock_guard<std::mutex> lock(p.mu);
  ProfRecord r{name, take_event(p), take_event(p), flops, bytes};
  hip_check(hipEventRecord(r.start, st), "hipEventRecord");
  p.records.push_back(r);
}

void prof_stop(hipStream_t st) {
  ProfState& p = prof_state();
  std::lock_guard<std::mutex> lock(p.mu);
  if (!p.records.empty()) (void)hipEventRecord(p.records.back().stop, st);
}

namespace {

// ---------------------------------------------------------------------------------
// Device buffer (RAII)
// ---------------------------------------------------------------------------------
struct DevBuf {
  void* ptr = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  DevBuf(DevBuf&& o) noexcept : ptr(o.ptr), bytes(o.bytes) {
    o.ptr = nullptr;
    o.bytes = 0;
  }
  DevBuf& operator=(DevBuf&& o) noexcept {
    if (this != &o) {
      release();
      ptr = o.ptr;
      bytes = o.bytes;
      o.ptr = nullptr;
      o.bytes = 0;
    }
    return *this;
  }
  ~DevBuf() { release(); }
  void release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
  }
  void ensure(size_t n) {
    if (n <= bytes && ptr) return;
    release();
    if (n == 0) return;
    hip_check(hipMalloc(&ptr, n), "hipMalloc");
    bytes = n;
  }
  template <class T>
  T* as() const {
    return reinterpret_cast<T*>(ptr);
  }
};

struct Param {
  std::string name;
  std::vector<int64_t> shape;
  std::vector<float> host;
  bool loaded = false;
  float max_abs = 0.f;  // max |value|, taken before the host copy is released
  DevBuf dev;  // reference layout on device
  int64_t numel() const {
    int64_t n = 1;
    for (auto s : shape) n *= s;
    return n;
  }
};

struct Shape3 {
  int d[3];
  int64_t vox() const { return (int64_t)d[0] * d[1] * d[2]; }
  bool operator==(const Shape3& o) const { return d[0] == o.d[0] && d[1] == o.d[1] && d[2] == o.d[2]; }
};

// Conv (+bias) + InstanceNorm (+activation); cin2 > 0 for the concat-free decoder conv.
struct ConvNorm {
  int cin1 = 0, cin2 = 0, cout = 0;
  int k[3] = {1, 1, 1}, s[3] = {1, 1, 1};
  bool act = true;
  int pw = -1, pb = -1, pg = -1, pbeta = -1;
  bool direct = false;
  bool direct_multi = false;  // 2 input channels: direct with split products if first
  bool first = false;   // reads the network input (kept in exact float32 products)
  bool split = false;   // packed for the split-fp16 kernel
  bool wino = false;    // packed for the Winograd split-fp16 kernel (within `split`)
  int level = 0;        // resolution level of the output (0 = full resolution)
  int arith = 0;        // split kernels' operand arithmetic (kArithSplit3 or kArithBf16)
  float scale = 1.f;    // power-of-two weight scale of the split packing
  DevBuf packed;
};

struct Upsample {
  int cin = 0, cout = 0;
  int k[3] = {2, 2, 2};
  int pw = -1, pb = -1;
  bool split = false;  // split-fp16 (or bf16) packing
  int level = 0;       // resolution level of the output
  int arith = 0;       // split kernels' operand arithmetic
  float scale = 1.f;
  DevBuf packed;
};

struct SegHead {
  int cin = 0, cout = 0;
  int pw = -1, pb = -1;
};

struct ResBlock {
  std::vector<ConvNorm> convs;  // basic: conv1 (act), conv2 (no act); bottleneck: 3 convs
  bool pool = false;
  int pool_k[3] = {1, 1, 1};
  bool proj = false;
  ConvNorm projc;
};

// Activation buffers for one (n, patch) shape.
struct Workspace {
  int n = 0;
  Shape3 in{};
  std::vector<std::unique_ptr<DevBuf>> bufs;
  DevBuf stats;   // per-tile InstanceNorm partials written by the conv epilogue
  size_t stats_bytes = 0;
  float* get(size_t i) { return bufs[i]->as<float>(); }
};

}  // namespace
}  // namespace nnx

struct nnx_model {
  // spec
  int arch = NNX_ARCH_PLAIN;
  int cin = 1, classes = 2, stages = 0;
  std::vector<int> features, ksz, strides, enc_count, dec_count, bottleneck;
  bool conv_bias = true, norm_affine = true;
  float eps = 1e-5f, slope = 0.01f;
  int stem_channels = 0;
  int precision = NNX_PRECISION_FP32;
  // params
  std::vector<nnx::Param> params;
  std::map<std::string, int> index;
  // graph
  std::vector<std::vector<nnx::ConvNorm>> enc;   // plain
  nnx::ConvNorm stem;                            // residual
  std::vector<std::vector<nnx::ResBlock>> res;   // residual
  std::vector<nnx::Upsample> up;
  std::vector<std::vector<nnx::ConvNorm>> dec;
  std::vector<nnx::SegHead> seg;
  bool finalized = false;
  // set while nnx_model_finalize uploads (it releases host copies as it goes): a call that
  // failed part-way leaves the model unusable
  bool finalize_failed = false;
  std::shared_ptr<nnx::Workspace> ws;
};

namespace nnx {
namespace {

int add_param(nnx_model* m, const std::string& name, std::vector<int64_t> shape) {
  require(m->index.find(name) == m->index.end(), "duplicate parameter " + name);
  Param p;
  p.name = name;
  p.shape = std::move(shape);
  m->params.push_back(std::move(p));
  const int id = (int)m->params.size() - 1;
  m->index[name] = id;
  return id;
}

void declare_convnorm(nnx_model* m, ConvNorm& c, const std::string& prefix, int level, int cin1,
                      int cin2, int cout, const int* k, const int* s, bool act, bool bias) {
  c.level = level;
  c.cin1 = cin1;
  c.cin2 = cin2;
  c.cout = cout;
  for (int i = 0; i < 3; ++i) {
    c.k[i] = k[i];
    c.s[i] = s[i];
  }
  c.act = act;
  c.pw = add_param(m, prefix + ".conv.weight", {cout, k[0], k[1], k[2], cin1 + cin2});
  if (bias) c.pb = add_param(m, prefix + ".conv.bias", {cout});
  if (m->norm_affine) {
    c.pg = add_param(m, prefix + ".norm.weight", {cout});
    c.pbeta = add_param(m, prefix + ".norm.bias", {cout});
  }
  const bool shape_ok = cin2 == 0 && k[0] == 3 && k[1] == 3 && k[2] == 3 && s[0] == 1 &&
                        s[1] == 1 && s[2] == 1 && cout % 4 == 0 && cout <= 64;
  c.direct = cin1 == 1 && shape_ok;
  // 2 or 4 input channels: the direct kernel with split products, for the network's first
  // convolution only (decided when packing, once the first convolution is known); with 4
  // channels 3.4 ms against 10.1 ms for the float32-product implicit GEMM per 32-view
  // 128^3 launch.
  c.direct_multi = (cin1 == 2 || cin1 == 4) && shape_ok;
}

const int kUnit[3] = {1, 1, 1};

void build_decoder(nnx_model* m) {
  const int S = m->stages;
  m->up.resize(S - 1);
  m->dec.resize(S - 1);
  m->seg.resize(S - 1);
  for (int d = 0; d < S - 1; ++d) {
    const int src = S - 1 - d;
    const int below = m->features[src];
    const int skip = m->features[src - 1];
    Upsample& u = m->up[d];
    u.level = src - 1;
    u.cin = below;
    u.cout = skip;
    for (int i = 0; i < 3; ++i) u.k[i] = m->strides[src * 3 + i];
    u.pw = add_param(m, "up" + std::to_string(d) + ".weight", {skip, u.k[0], u.k[1], u.k[2], below});
    if (m->conv_bias) u.pb = add_param(m, "up" + std::to_string(d) + ".bias", {skip});
    m->dec[d].resize(m->dec_count[d]);
    for (int j = 0; j < m->dec_count[d]; ++j) {
      declare_convnorm(m, m->dec[d][j], "dec" + std::to_string(d) + ".block" + std::to_string(j),
                       src - 1, j == 0 ? skip : skip, j == 0 ? skip : 0, skip, &m->ksz[(src - 1) * 3],
                       kUnit, true, m->conv_bias);
    }
    SegHead& sh = m->seg[d];
    sh.cin = skip;
    sh.cout = m->classes;
    sh.pw = add_param(m, "seg" + std::to_string(d) + ".weight", {m->classes, 1, 1, 1, skip});
    sh.pb = add_param(m, "seg" + std::to_string(d) + ".bias", {m->classes});
  }
}

void build_graph(nnx_model* m) {
  const int S = m->stages;
  if (m->arch == NNX_ARCH_PLAIN) {
    m->enc.resize(S);
    int cin = m->cin;
    for (int s = 0; s < S; ++s) {
      m->enc[s].resize(m->enc_count[s]);
      for (int j = 0; j < m->enc_count[s]; ++j) {
        declare_convnorm(m, m->enc[s][j], "enc" + std::to_string(s) + ".block" + std::to_string(j),
                         s, j == 0 ? cin : m->features[s], 0, m->features[s], &m->ksz[s * 3],
                         j == 0 ? &m->strides[s * 3] : kUnit, true, m->conv_bias);
      }
      cin = m->features[s];
    }
  } else {
    const int stem_ch = m->stem_channels > 0 ? m->stem_channels : m->features[0];
    declare_convnorm(m, m->stem, "stem", 0, m->cin, 0, stem_ch, &m->ksz[0], kUnit, true, m->conv_bias);
    m->res.resize(S);
    int cin = stem_ch;
    for (int s = 0; s < S; ++s) {
      m->res[s].resize(m->enc_count[s]);
      for (int b = 0; b < m->enc_count[s]; ++b) {
        ResBlock& rb = m->res[s][b];
        const int bin = b == 0 ? cin : m->features[s];
        const int bout = m->features[s];
        const int* stride = b == 0 ? &m->strides[s * 3] : kUnit;
        const std::string pre = "res" + std::to_string(s) + ".block" + std::to_string(b);
        if (m->bottleneck.empty()) {
          rb.convs.resize(2);
          declare_convnorm(m, rb.convs[0], pre + ".conv1", s, bin, 0, bout, &m->ksz[s * 3], stride,
                           true, m->conv_bias);
          declare_convnorm(m, rb.convs[1], pre + ".conv2", s, bout, 0, bout, &m->ksz[s * 3], kUnit,
                           false, m->conv_bias);
        } else {
          const int bc = m->bottleneck[s];
          rb.convs.resize(3);
          declare_convnorm(m, rb.convs[0], pre + ".conv1", s, bin, 0, bc, kUnit, kUnit, true,
                           m->conv_bias);
          declare_convnorm(m, rb.convs[1], pre + ".conv2", s, bc, 0, bc, &m->ksz[s * 3], stride, true,
                           m->conv_bias);
          declare_convnorm(m, rb.convs[2], pre + ".conv3", s, bc, 0, bout, kUnit, kUnit, false,
                           m->conv_bias);
        }
        rb.pool = !(stride[0] == 1 && stride[1] == 1 && stride[2] == 1);
        for (int i = 0; i < 3; ++i) rb.pool_k[i] = stride[i];
        rb.proj = bin != bout;
        if (rb.proj)
          declare_convnorm(m, rb.projc, pre + ".proj", s, bin, 0, bout, kUnit, kUnit, false, false);
      }
      cin = m->features[s];
    }
  }
  build_decoder(m);
}

const float* pdev(const nnx_model* m, int id) {
  return id < 0 ? nullptr : m->params[id].dev.as<float>();
}

// The split kernels' operand arithmetic of a layer at resolution `level`: bf16 in the bf16
// precision, and in the mixed bf16 precision below full resolution; fp16-split otherwise.
int layer_arith(const nnx_model* m, int level) {
  if (m->precision == NNX_PRECISION_BF16) return kArithBf16;
  if (m->precision == NNX_PRECISION_BF16_MIXED && level > 0) return kArithBf16;
  return kArithSplit3;
}
bool uses_split_kernels(const nnx_model* m) {
  return m->precision != NNX_PRECISION_FP32;
}
// Precisions whose first convolution with 1 or 2 input channels takes split products with a
// per-tile input scale (the all-bf16 precision keeps float32 products there).
bool split_first_conv(const nnx_model* m) {
  return m->precision == NNX_PRECISION_FP32_SPLIT || m->precision == NNX_PRECISION_BF16_MIXED;
}

// The stride-1 3x3x3 fp16-split layers with C_out % 32 == 0 and 16-channel input blocks run
// on the Winograd kernel (fewer fp16 MFMA products per output, so less energy per output
// under the chip's power cap); NNX_CONV_ALGO=direct keeps every layer on the direct implicit
// GEMM (read when a model's weights are packed, for comparisons).
bool winograd_enabled() {
  const char* v = std::getenv("NNX_CONV_ALGO");
  return !(v && std::string(v) == "direct");
}

void pack_convnorm(nnx_model* m, ConvNorm& c, hipStream_t st) {
  if (c.first && c.direct_multi && split_first_conv(m)) c.direct = true;
  if (c.direct) {
    // the direct kernel reads the reference layout; split products in the fp32-split and
    // mixed bf16 precisions (the bf16 precision keeps float32 products for the first
    // convolution)
    c.split = split_first_conv(m);
    c.scale = c.split ? split_weight_scale(m->params[c.pw].max_abs) : 0.f;
    return;
  }
  // Split-fp16 (or bf16) products for the hidden convolutions with >= 8 taps (a tap group
  // holds 4 taps; 1x1x1 convolutions would waste 3/4 of it).  A first convolution that
  // reaches this point (more than 2 input channels, or any first convolution in bf16) reads
  // the raw network input, whose range is not normalised, so it keeps float32 products;
  // first convolutions with 1 or 2 input channels took the direct kernel above (split
  // products with a per-tile input scale in the fp32-split precision).
  const int taps = c.k[0] * c.k[1] * c.k[2];
  c.split = uses_split_kernels(m) && !c.first && taps >= 8 && conv_x3_supported(c.k, c.s, c.cout);
  c.arith = layer_arith(m, c.level);
  if (c.split && c.arith == kArithSplit3 && winograd_enabled()) {
    const int probe[3] = {16, 16, 16};
    c.wino = conv_wino_supported(make_conv_geom(1, probe, c.k, c.s), c.cin1, c.cin2, c.cout);
  }
  if (c.wino) {
    c.scale = wino_weight_scale(m->params[c.pw].max_abs);
    c.packed.ensure((size_t)conv_wino_packed_bytes(c.cout, c.cin1, c.cin2));
    conv_wino_pack_weight(pdev(m, c.pw), c.cout, c.cin1, c.cin2, c.scale, c.packed.ptr, st);
    return;
  }
  if (c.split) {
    c.scale = split_weight_scale(m->params[c.pw].max_abs);
    c.packed.ensure((size_t)conv_x3_packed_bytes(c.cout, c.k, c.cin1, c.cin2));
    conv_x3_pack_weight(pdev(m, c.pw), c.cout, c.k, c.cin1, c.cin2, c.scale, c.packed.ptr, st,
                        c.arith);
    return;
  }
  const int64_t n = conv_packed_floats(c.cout, c.k, c.cin1, c.cin2);
  c.packed.ensure((size_t)n * sizeof(float));
  conv_pack_weight(pdev(m, c.pw), c.cout, c.k, c.cin1, c.cin2, c.packed.as<float>(), st);
}

// ---------------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------------
Shape3 conv_out(const Shape3& in, const ConvNorm& c) {
  Shape3 o;
  for (int i = 0; i < 3; ++i) o.d[i] = (in.d[i] + 2 * (c.k[i] / 2) - c.k[i]) / c.s[i] + 1;
  return o;
}

// Layer checks (NNX_CHECK_LAYERS=1 in the environment, or nnx_set_layer_checks(1)): after
// every convolution, transposed convolution and head the stream is synchronised and the
// layer's output is scanned for non-finite values; the first such layer fails the forward
// with its parameter name and the batch geometry.  A diagnostic, off by default (it
// serialises the forward): the host turns it on to name the layer when a forward has
// produced non-finite logits.
std::atomic<bool> g_layer_checks{false};

bool layer_checks_enabled() {
  static const bool env = [] {
    const char* v = std::getenv("NNX_CHECK_LAYERS");
    return v != nullptr && v[0] == '1';
  }();
  return env || g_layer_checks.load(std::memory_order_relaxed);
}

void check_layer(const std::string& name, const float* buf, int64_t n, int batch, hipStream_t st) {
  static DevBuf* counter = new DevBuf();  // lives until process exit
  counter->ensure(sizeof(unsigned int));
  count_nonfinite(buf, n, counter->as<unsigned int>(), st);
  unsigned int bad = 0;
  hip_check(hipMemcpyAsync(&bad, counter->ptr, sizeof(bad), hipMemcpyDeviceToHost, st),
            "layer check copy");
  hip_check(hipStreamSynchronize(st), "layer check synchronize");
  if (bad)
    fail(NNX_ERR_NONFINITE, "layer check: " + std::to_string(bad) + " non-finite values of " +
                                std::to_string(n) + " in the output of " + name + " (batch " +
                                std::to_string(batch) + ")");
}

struct Planner {
  // During planning, records buffer sizes; during execution, hands out the same buffers.
  std::vector<size_t> sizes;
  size_t stats = 0;
  size_t next = 0;
  bool planning = true;
  Workspace* ws = nullptr;
  int batch = 1;
  float* take(size_t floats) {
    if (planning) {
      // kernels address a batch item's voxels with 32-bit offsets (whole-batch offsets are
      // 64-bit), so one item of an activation stays below 2^31 elements
      require(floats / (size_t)batch < ((size_t)1 << 31),
              "a network activation exceeds 2^31 elements per batch item; use a smaller patch");
      sizes.push_back(floats * sizeof(float));
      return nullptr;
    }
    require(next < ws->bufs.size(), "workspace plan mismatch");
    return ws->get(next++);
  }
};

// An activation as its consumer sees it: the buffer, plus the InstanceNorm (+ LeakyReLU)
// still to be applied to it when the producer deferred its apply pass to the consumer.
struct Act {
  const float* data = nullptr;
  PendingNorm norm;
};


struct Runner {
  nnx_model* m;
  Planner* plan;
  hipStream_t st;
  int n;

  // Conv + InstanceNorm (+ LeakyReLU).  With `defer` (every consumer of the output is a
  // convolution or the segmentation head, which normalise on load) the apply pass is
  // skipped and the output carries its parameters; otherwise it is applied in place
  // (with the residual addition for a residual block's last convolution).
  Act convnorm(const ConvNorm& c, const Act& x1, const Act& x2, const Shape3& in, float* out,
               const Shape3& outs, const float* residual, bool defer) {
    const int64_t vox = outs.vox();
    // A residual block's last ConvNorm has no activation of its own; LeakyReLU follows the
    // residual addition (ResidualBlock.__call__), fused into the same apply pass.
    const bool act = c.act || residual != nullptr;
    require(!(defer && residual), "a residual sum cannot be deferred");
    float4* params = reinterpret_cast<float4*>(plan->take((size_t)n * c.cout * 4));
    Act result;
    result.data = out;
    if (defer) result.norm = PendingNorm{params, act, m->slope};
    if (c.direct) {
      // the direct kernel writes per-block statistics of its output
      require(!x1.norm.params, "the one-channel convolution reads the network input");
      const int tiles = conv_direct_stats_tiles(in.d, c.split);
      if (plan->planning) {
        plan->stats = std::max(plan->stats, (size_t)n * tiles * c.cout * sizeof(float4));
        return result;
      }
      float4* stats = plan->ws->stats.as<float4>();
      conv3d_direct_cin1(x1.data, pdev(m, c.pw), pdev(m, c.pb), out, n, in.d, c.cout, st, stats,
                         c.split ? c.scale : 0.f, c.cin1);
      instnorm_merge_partials(stats, tiles, n, vox, c.cout, pdev(m, c.pg), pdev(m, c.pbeta),
                              m->eps, params, st);
      if (!defer)
        instnorm_apply_params(out, out, n, vox, c.cout, params, nullptr, act, m->slope, residual,
                              st);
      if (layer_checks_enabled())
        check_layer(m->params[c.pw].name, out, (int64_t)n * vox * c.cout, n, st);
      return result;
    }
    // Implicit GEMM: the epilogue writes per-tile statistics, so the norm never re-reads the
    // tensor for them.
    const ConvGeom g = make_conv_geom(n, in.d, c.k, c.s);
    const int tiles = c.wino    ? conv_wino_stats_tiles(g)
                      : c.split ? conv_x3_stats_tiles(g, c.cout)
                                : conv_stats_tiles(g, c.cout, c.cin1, c.cin2);
    if (plan->planning) {
      plan->stats = std::max(plan->stats, (size_t)n * tiles * c.cout * sizeof(float4));
      return result;
    }
    float4* stats = plan->ws->stats.as<float4>();
    if (c.wino)
      conv3d_wino(x1.data, c.cin1, x2.data, c.cin2, c.packed.ptr, c.scale, pdev(m, c.pb), out, g,
                  c.cout, st, stats, x1.norm, x2.norm);
    else if (c.split)
      conv3d_x3(x1.data, c.cin1, x2.data, c.cin2, c.packed.ptr, c.scale, pdev(m, c.pb), out, g,
                c.cout, st, stats, x1.norm, x2.norm, c.arith);
    else
      conv3d_igemm(x1.data, c.cin1, x2.data, c.cin2, c.packed.as<float>(), pdev(m, c.pb), out, g,
                   c.cout, st, stats, x1.norm, x2.norm);
    instnorm_merge_partials(stats, tiles, n, vox, c.cout, pdev(m, c.pg), pdev(m, c.pbeta), m->eps,
                            params, st);
    if (!defer)
      instnorm_apply_params(out, out, n, vox, c.cout, params, nullptr, act, m->slope, residual,
                            st);
    if (layer_checks_enabled())
      check_layer(m->params[c.pw].name, out, (int64_t)n * vox * c.cout, n, st);
    return result;
  }

  // *outs receives the output's spatial shape.
  Act run_convnorm(const ConvNorm& c, const Act& x1, const Act& x2, const Shape3& in,
                   Shape3* outs, bool defer, const float* residual = nullptr) {
    *outs = conv_out(in, c);
    float* out = plan->take((size_t)n * outs->vox() * c.cout);
    return convnorm(c, x1, x2, in, out, *outs, residual, defer);
  }

  // The decoder.  Its last stage feeds the segmentation head, which normalises on load;
  // every other stage's last output feeds a transposed convolution, which normalises on load
  // when split and otherwise takes an applied tensor.
  void decode(std::vector<Act>& skips, std::vector<Shape3>& skip_shapes, float* d_out) {
    const int S = m->stages;
    Act hidden = skips[S - 1];
    Shape3 hs = skip_shapes[S - 1];
    for (int d = 0; d < S - 1; ++d) {
      const int src = S - 1 - d;
      const Upsample& u = m->up[d];
      require(!hidden.norm.params || u.split,
              "only the split transposed convolution normalises its input on load");
      Shape3 us;
      for (int i = 0; i < 3; ++i) us.d[i] = hs.d[i] * u.k[i];
      const Shape3& ss = skip_shapes[src - 1];
      float* upbuf = plan->take((size_t)n * us.vox() * u.cout);
      if (!plan->planning) {
        if (u.split)
          tconv3d_x3(hidden.data, u.cin, u.packed.ptr, u.scale, pdev(m, u.pb), upbuf, n, hs.d,
                     u.cout, u.k, st, u.arith, hidden.norm);
        else
          tconv3d_gemm(hidden.data, u.cin, u.packed.as<float>(), pdev(m, u.pb), upbuf, n, hs.d,
                       u.cout, u.k, st);
        if (layer_checks_enabled())
          check_layer(m->params[u.pw].name, upbuf, (int64_t)n * us.vox() * u.cout, n, st);
      }
      if (!(us == ss)) {
        // patch not divisible by the total stride: centre crop / zero pad the upsampled
        // tensor to the skip's size (_match_spatial, src/nnunet_mlx/model/network.py:898-916)
        float* matched = plan->take((size_t)n * ss.vox() * u.cout);
        if (!plan->planning) match_spatial(upbuf, us.d, matched, ss.d, n, u.cout, st);
        upbuf = matched;
      }
      Shape3 cur = ss;
      Act a;
      a.data = upbuf;
      const size_t nb = m->dec[d].size();
      for (size_t j = 0; j < nb; ++j) {
        Shape3 o;
        // the stage's output feeds the next transposed convolution (which normalises on
        // load when split and the stage's voxels fill its row tiles) or, for the last
        // stage, the segmentation head
        const bool defer = j + 1 < nb || d == S - 2 || (m->up[d + 1].split && tconv_norm_on_load(ss.d));
        a = run_convnorm(m->dec[d][j], a, j == 0 ? skips[src - 1] : Act{}, cur, &o, defer);
        cur = o;
      }
      hidden = a;
      hs = cur;
    }
    const SegHead& sh = m->seg[S - 2];
    if (!plan->planning) {
      conv1x1(hidden.data, sh.cin, pdev(m, sh.pw), pdev(m, sh.pb), d_out, (int64_t)n * hs.vox(),
              sh.cout, st, hidden.norm, hs.vox());
      if (layer_checks_enabled())
        check_layer(m->params[sh.pw].name, d_out, (int64_t)n * hs.vox() * sh.cout, n, st);
    }
  }

  void forward_plain(const float* x, const Shape3& in, float* d_out) {
    const int S = m->stages;
    std::vector<Act> skips(S);
    std::vector<Shape3> shapes(S);
    Act h;
    h.data = x;
    Shape3 cur = in;
    for (int s = 0; s < S; ++s) {
      const size_t nb = m->enc[s].size();
      for (size_t j = 0; j < nb; ++j) {
        Shape3 o;
        // the bottleneck's output feeds the first transposed convolution, which normalises
        // on load when split and the bottleneck's voxels fill its row tiles
        const bool last = s == S - 1 && j + 1 == nb;
        const bool defer = !last || (S > 1 && m->up[0].split &&
                                     tconv_norm_on_load(conv_out(cur, m->enc[s][j]).d));
        h = run_convnorm(m->enc[s][j], h, Act{}, cur, &o, defer);
        cur = o;
      }
      skips[s] = h;
      shapes[s] = cur;
    }
    decode(skips, shapes, d_out);
  }

  // Residual encoder: block outputs (residual sums) and the stem are applied tensors; the
  // inner convolutions of a block defer to the next convolution of the block.
  void forward_residual(const float* x, const Shape3& in, float* d_out) {
    const int S = m->stages;
    std::vector<Act> skips(S);
    std::vector<Shape3> shapes(S);
    Shape3 cur;
    Act xin;
    xin.data = x;
    Act h = run_convnorm(m->stem, xin, Act{}, in, &cur, false);
    for (int s = 0; s < S; ++s) {
      for (auto& rb : m->res[s]) {
        // skip path: pool (stride) then 1x1 projection (channel change)
        const float* residual = h.data;
        Shape3 rs = cur;
        const int cin = rb.convs[0].cin1;
        if (rb.pool) {
          for (int i = 0; i < 3; ++i) {
            require(cur.d[i] % rb.pool_k[i] == 0,
                    "residual block input size must be divisible by its stride");
            rs.d[i] = cur.d[i] / rb.pool_k[i];
          }
          float* pooled = plan->take((size_t)n * rs.vox() * cin);
          if (!plan->planning) {
            avgpool3d(h.data, pooled, n, cur.d, cin, rb.pool_k, st);
            if (layer_checks_enabled())
              check_layer(m->params[rb.convs[0].pw].name + " (shortcut pool)", pooled,
                          (int64_t)n * rs.vox() * cin, n, st);
          }
          residual = pooled;
        }
        if (rb.proj) {
          Shape3 ps;
          Act r;
          r.data = residual;
          residual = run_convnorm(rb.projc, r, Act{}, rs, &ps, false).data;
          rs = ps;
        }
        Act a = h;
        Shape3 as = cur;
        for (size_t j = 0; j < rb.convs.size(); ++j) {
          Shape3 o;
          const bool last = j + 1 == rb.convs.size();
          if (last) {
            o = conv_out(as, rb.convs[j]);
            require(o == rs, "residual branch and shortcut shapes differ");
          }
          // the last conv has no activation of its own: LeakyReLU follows the residual add
          a = run_convnorm(rb.convs[j], a, Act{}, as, &o, !last, last ? residual : nullptr);
          as = o;
        }
        h = a;
        cur = as;
      }
      skips[s] = h;
      shapes[s] = cur;
    }
    decode(skips, shapes, d_out);
  }

  void forward(const float* x, const Shape3& in, float* out) {
    if (m->arch == NNX_ARCH_PLAIN)
      forward_plain(x, in, out);
    else
      forward_residual(x, in, out);
  }
};

void ensure_workspace(nnx_model* m, int n, const Shape3& in) {
  if (!m->ws) m->ws = std::make_shared<Workspace>();
  Workspace& ws = *m->ws;
  Planner plan;
  plan.planning = true;
  plan.batch = n;
  Runner r{m, &plan, nullptr, n};
  r.forward(nullptr, in, nullptr);
  // grow every slot to the largest need seen so far (folds sharing one workspace may
  // differ in channel counts only if they differ in architecture; sizes are per slot)
  if (ws.bufs.size() < plan.sizes.size()) ws.bufs.resize(plan.sizes.size());
  for (size_t i = 0; i < plan.sizes.size(); ++i) {
    if (!ws.bufs[i]) ws.bufs[i] = std::make_unique<DevBuf>();
    ws.bufs[i]->ensure(plan.sizes[i]);
  }
  if (plan.stats > ws.stats_bytes) {
    ws.stats.ensure(plan.stats);
    ws.stats_bytes = plan.stats;
  }
  ws.n = n;
  ws.in = in;
}

void run_forward(nnx_model* m, const float* x, float* out, int n, const int* spatial,
                 hipStream_t st) {
  require(m != nullptr, "model must not be null");
  require(m->finalized, "nnx_model_finalize must be called before nnx_forward");
  require(x && out, "forward pointers must not be null");
  require(n >= 1, "forward batch must be positive");
  Shape3 in{{spatial[0], spatial[1], spatial[2]}};
  for (int i = 0; i < 3; ++i) require(in.d[i] >= 1, "forward spatial size must be positive");
  ensure_workspace(m, n, in);
  Planner plan;
  plan.planning = false;
  plan.ws = m->ws.get();
  Runner r{m, &plan, st, n};
  r.forward(x, in, out);
}

// ---------------------------------------------------------------------------------
// Sliding window
// ---------------------------------------------------------------------------------
struct SwCache {
  std::mutex mu;
  DevBuf acc, norm, total, batch_in, batch_out, counter;
};

SwCache& sw_cache() {
  static SwCache* c = new SwCache();  // intentionally leaked: lives until process exit
  return *c;
}

struct ModelForward {
  static int call(void* user, const float* in, float* out, int n, const int* spatial,
                  void* stream) {
    run_forward(reinterpret_cast<nnx_model*>(user), in, out, n, spatial, as_stream(stream));
    return NNX_OK;
  }
};

// a * b, refused when the product leaves [0, 2^62) (every buffer size below is one)
int64_t sw_product(int64_t a, int64_t b, const char* what) {
  int64_t r = 0;
  require(!__builtin_mul_overflow(a, b, &r) && r >= 0 && r < (int64_t(1) << 62),
          std::string("sliding-window ") + what + " too large");
  return r;
}

void validate_sw(const nnx_sw_config* c) {
  require(c != nullptr, "sliding-window config must not be null");
  require(c->channels >= 1, "sliding-window input needs at least one channel");
  require(c->num_classes >= 1, "sliding-window inference requires at least one output channel");
  require(c->channels <= 65535 && c->num_classes <= 65535,
          "sliding-window channels and classes are limited to 65535");
  require(c->accumulation == NNX_ACCUM_F32 || c->accumulation == NNX_ACCUM_NNUNET_F16,
          "unsupported sliding-window accumulation");
  require(c->ntiles >= 1 && c->tile_offsets, "sliding window needs at least one tile");
  require(c->nviews >= 1 && c->nviews <= 8 && c->view_flips, "between 1 and 8 views");
  require(c->d_gaussian != nullptr, "gaussian map must not be null");
  require(c->tiles_per_batch >= 1, "tiles_per_batch must be positive");
  for (int i = 0; i < 3; ++i) {
    require(c->size[i] >= 1 && c->patch[i] >= 1, "invalid volume or patch size");
    require(c->padded[i] < (int64_t(1) << 31), "volume dimensions are limited to 2^31 - 1");
    require(c->pad_before[i] >= 0 && c->padded[i] >= c->size[i] + c->pad_before[i],
            "invalid minimum padding");
    require(c->padded[i] >= c->patch[i], "padded image dimension is smaller than the patch");
  }
  // every buffer the run sizes: accumulators (padded volume x classes), fold total (crop x
  // classes), a batch of views in and out (patch x channels or classes)
  const int64_t esz = c->accumulation == NNX_ACCUM_NNUNET_F16 ? 2 : 4;
  const int64_t padded_vox = sw_product(sw_product(c->padded[0], c->padded[1], "volume"),
                                        c->padded[2], "volume");
  sw_product(sw_product(padded_vox, c->num_classes, "volume"), esz, "volume");
  const int64_t patch_vox =
      sw_product(sw_product(c->patch[0], c->patch[1], "patch"), c->patch[2], "patch");
  const int64_t views = sw_product(std::min(c->tiles_per_batch, c->ntiles), c->nviews, "batch");
  sw_product(sw_product(views, patch_vox, "batch"),
             (int64_t)std::max(c->channels, c->num_classes) * 4, "batch");
  for (int t = 0; t < c->ntiles; ++t)
    for (int i = 0; i < 3; ++i) {
      const int64_t o = c->tile_offsets[t * 3 + i];
      require(o >= 0 && o + c->patch[i] <= c->padded[i], "tile offset outside the padded volume");
    }
}

void sw_run(nnx_forward_fn const* forwards, void* const* users, int nfolds, const nnx_sw_config* c,
            const float* vol, void* logits, uint16_t* labels, hipStream_t st) {
  validate_sw(c);
  require(nfolds >= 1, "fold inference requires at least one model");
  require(vol != nullptr, "volume must not be null");
  SwCache& cache = sw_cache();
  std::lock_guard<std::mutex> lock(cache.mu);
  const int K = c->num_classes;
  const size_t esz = c->accumulation == NNX_ACCUM_NNUNET_F16 ? 2 : 4;
  const int64_t padded_vox = c->padded[0] * c->padded[1] * c->padded[2];
  const int64_t crop_vox = c->size[0] * c->size[1] * c->size[2];
  const int64_t patch_vox = (int64_t)c->patch[0] * c->patch[1] * c->patch[2];
  const int tpb = std::min(c->tiles_per_batch, c->ntiles);
  cache.acc.ensure((size_t)padded_vox * K * esz);
  cache.norm.ensure((size_t)padded_vox * esz);
  cache.total.ensure((size_t)crop_vox * K * esz);
  cache.batch_in.ensure((size_t)tpb * c->nviews * patch_vox * c->channels * sizeof(float));
  cache.batch_out.ensure((size_t)tpb * c->nviews * patch_vox * K * sizeof(float));
  cache.counter.ensure(sizeof(unsigned int));
  float* bin = cache.batch_in.as<float>();
  float* bout = cache.batch_out.as<float>();
  const int crop_lo[3] = {c->pad_before[0], c->pad_before[1], c->pad_before[2]};
  for (int f = 0; f < nfolds; ++f) {
    require(forwards[f] != nullptr, "forward callback must not be null");
    fill_zero(cache.acc.ptr, (size_t)padded_vox * K * esz, st);
    fill_zero(cache.norm.ptr, (size_t)padded_vox * esz, st);
    for (int t0 = 0; t0 < c->ntiles; t0 += tpb) {
      const int nt = std::min(tpb, c->ntiles - t0);
      for (int i = 0; i < nt; ++i)
        sw_gather_flip(vol, c->channels, c->size, c->pad_before, &c->tile_offsets[(t0 + i) * 3],
                       c->patch, c->view_flips, c->nviews,
                       bin + (int64_t)i * c->nviews * patch_vox * c->channels, st);
      const int rc = forwards[f](users[f], bin, bout, nt * c->nviews, c->patch, st);
      if (rc != NNX_OK) fail(rc, "forward callback failed: " + g_last_error);
      for (int i = 0; i < nt; ++i)
        sw_accumulate(bout + (int64_t)i * c->nviews * patch_vox * K, c->nviews, c->view_flips, K,
                      c->patch, c->d_gaussian, &c->tile_offsets[(t0 + i) * 3], c->padded,
                      c->accumulation, cache.acc.ptr, cache.norm.ptr, st);
    }
    sw_fold_add(cache.acc.ptr, cache.norm.ptr, K, c->padded, crop_lo, c->size, c->accumulation,
                f == 0, cache.total.ptr, st);
  }
  unsigned int* counter = cache.counter.as<unsigned int>();
  sw_fold_finalize(cache.total.ptr, K, crop_vox, nfolds, c->accumulation, logits, labels, counter,
                   st);
  unsigned int invalid = 0;
  hip_check(hipMemcpyAsync(&invalid, counter, sizeof(invalid), hipMemcpyDeviceToHost, st),
            "copy invalid count");
  hip_check(hipStreamSynchronize(st), "sliding-window synchronize");
  if (invalid) fail(NNX_ERR_NONFINITE, "sliding-window inference produced non-finite logits");
}

}  // namespace
}  // namespace nnx

// =====================================================================================
// extern "C" boundary
// =====================================================================================
using namespace nnx;

extern "C" {

const char* nnx_last_error(void) { return g_last_error.c_str(); }

const char* nnx_version(void) { return "nnunet-hip 0.1.0 gfx950"; }

int nnx_model_create(const nnx_spec* spec, nnx_model** out) {
  return guarded([&] {
    require(spec && out, "spec and output pointers must not be null");
    *out = nullptr;
    require(spec->spatial_dims == 3, "only three-dimensional networks run on the HIP path");
    require(spec->arch == NNX_ARCH_PLAIN || spec->arch == NNX_ARCH_RESIDUAL,
            "unsupported network architecture");
    require(spec->precision == NNX_PRECISION_FP32 || spec->precision == NNX_PRECISION_FP32_SPLIT ||
                spec->precision == NNX_PRECISION_BF16 ||
                spec->precision == NNX_PRECISION_BF16_MIXED,
            "unsupported precision");
    // upper bounds: no network that could run exceeds them (every normalised layer is
    // limited to 1024 channels), and they keep the graph and its parameter sizes small
    constexpr int kMaxWidth = 1024, kMaxStages = 16, kMaxKernel = 15, kMaxStride = 16,
                  kMaxConvs = 64;
    require(spec->input_channels >= 1 && spec->num_classes >= 1,
            "network needs input channels and at least one output");
    require(spec->input_channels <= kMaxWidth && spec->num_classes <= kMaxWidth,
            "input channels and classes are limited to 1024");
    require(spec->n_stages >= 2, "network needs at least two stages");
    require(spec->n_stages <= kMaxStages, "network has more than 16 stages");
    require(spec->stem_channels <= kMaxWidth, "stem channels are limited to 1024");
    require(spec->features && spec->kernel_sizes && spec->strides && spec->encoder_convs &&
                spec->decoder_convs,
            "spec arrays must not be null");
    require(spec->norm_eps > 0.f, "normalization epsilon must be positive");
    require(spec->leaky_slope >= 0.f && spec->leaky_slope <= 1.f,
            "LeakyReLU negative_slope must be in [0, 1]");
    auto m = std::make_unique<nnx_model>();
    m->arch = spec->arch;
    m->cin = spec->input_channels;
    m->classes = spec->num_classes;
    m->stages = spec->n_stages;
    const int S = spec->n_stages;
    m->features.assign(spec->features, spec->features + S);
    m->ksz.assign(spec->kernel_sizes, spec->kernel_sizes + 3 * S);
    m->strides.assign(spec->strides, spec->strides + 3 * S);
    m->enc_count.assign(spec->encoder_convs, spec->encoder_convs + S);
    m->dec_count.assign(spec->decoder_convs, spec->decoder_convs + S - 1);
    if (spec->arch == NNX_ARCH_RESIDUAL && spec->bottleneck_channels)
      m->bottleneck.assign(spec->bottleneck_channels, spec->bottleneck_channels + S);
    for (int v : m->features)
      require(v >= 1 && v <= kMaxWidth, "features must lie in 1..1024");
    for (int v : m->ksz)
      require(v >= 1 && v % 2 == 1 && v <= kMaxKernel,
              "only odd convolution kernels of 1..15 are supported");
    for (int v : m->strides) require(v >= 1 && v <= kMaxStride, "strides must lie in 1..16");
    for (int v : m->enc_count)
      require(v >= 1 && v <= kMaxConvs, "encoder counts must lie in 1..64");
    for (int v : m->dec_count)
      require(v >= 1 && v <= kMaxConvs, "decoder counts must lie in 1..64");
    for (int v : m->bottleneck)
      require(v >= 1 && v <= kMaxWidth, "bottleneck channels must lie in 1..1024");
    m->conv_bias = spec->conv_bias != 0;
    m->norm_affine = spec->norm_affine != 0;
    m->eps = spec->norm_eps;
    m->slope = spec->leaky_slope;
    m->stem_channels = spec->stem_channels;
    m->precision = spec->precision;
    build_graph(m.get());
    if (m->arch == NNX_ARCH_PLAIN)
      m->enc[0][0].first = true;
    else
      m->stem.first = true;
    *out = m.release();
  });
}

int nnx_model_param_count(const nnx_model* model, int* count) {
  return guarded([&] {
    require(model && count, "null argument");
    *count = (int)model->params.size();
  });
}

int nnx_model_param_info(const nnx_model* model, int index, const char** name, int* ndim,
                         int64_t* shape) {
  return guarded([&] {
    require(model && name && ndim && shape, "null argument");
    require(index >= 0 && index < (int)model->params.size(), "parameter index out of range");
    const Param& p = model->params[index];
    *name = p.name.c_str();
    *ndim = (int)p.shape.size();
    for (size_t i = 0; i < p.shape.size(); ++i) shape[i] = p.shape[i];
  });
}

int nnx_model_load_param(nnx_model* model, const char* name, const float* host,
                         const int64_t* shape, int ndim) {
  return guarded([&] {
    require(model && name && host && shape, "null argument");
    require(!model->finalized, "parameters cannot change after nnx_model_finalize");
    auto it = model->index.find(name);
    if (it == model->index.end()) fail(NNX_ERR_STATE, std::string("unexpected parameter ") + name);
    Param& p = model->params[it->second];
    if (p.loaded) fail(NNX_ERR_STATE, std::string("parameter loaded twice: ") + name);
    bool same = ndim == (int)p.shape.size();
    for (int i = 0; same && i < ndim; ++i) same = shape[i] == p.shape[i];
    if (!same) {
      std::string want = "(";
      for (size_t i = 0; i < p.shape.size(); ++i) want += std::to_string(p.shape[i]) + (i + 1 < p.shape.size() ? "," : "");
      fail(NNX_ERR_INVALID, std::string("parameter ") + name + " has the wrong shape; expected " + want + ")");
    }
    const int64_t n = p.numel();
    for (int64_t i = 0; i < n; ++i)
      if (!std::isfinite(host[i])) fail(NNX_ERR_INVALID, std::string("model tensor '") + name + "' is non-finite");
    p.host.assign(host, host + n);
    p.loaded = true;
  });
}

int nnx_model_finalize(nnx_model* model) {
  return guarded([&] {
    require(model != nullptr, "model must not be null");
    require(!model->finalized, "model already finalized");
    std::string missing;
    for (const Param& p : model->params)
      if (!p.loaded) missing += (missing.empty() ? "" : ", ") + p.name;
    if (!missing.empty()) fail(NNX_ERR_STATE, "missing parameters: " + missing);
    require(!model->finalize_failed,
            "an earlier nnx_model_finalize failed part-way; destroy and rebuild the model");
    model->finalize_failed = true;
    for (Param& p : model->params) {
      for (float v : p.host) p.max_abs = std::max(p.max_abs, std::fabs(v));
      p.dev.ensure((size_t)p.numel() * sizeof(float));
      hip_check(hipMemcpy(p.dev.ptr, p.host.data(), (size_t)p.numel() * sizeof(float),
                          hipMemcpyHostToDevice),
                "upload parameter");
      std::vector<float>().swap(p.host);
    }
    hipStream_t st = nullptr;
    if (model->arch == NNX_ARCH_PLAIN) {
      for (auto& stage : model->enc)
        for (auto& c : stage) pack_convnorm(model, c, st);
    } else {
      pack_convnorm(model, model->stem, st);
      for (auto& stage : model->res)
        for (auto& rb : stage) {
          for (auto& c : rb.convs) pack_convnorm(model, c, st);
          if (rb.proj) pack_convnorm(model, rb.projc, st);
        }
    }
    for (auto& stage : model->dec)
      for (auto& c : stage) pack_convnorm(model, c, st);
    for (auto& u : model->up) {
      u.split = uses_split_kernels(model);
      u.arith = layer_arith(model, u.level);
      if (u.split) {
        u.scale = split_weight_scale(model->params[u.pw].max_abs);
        u.packed.ensure((size_t)tconv_x3_packed_bytes(u.cout, u.k, u.cin));
        tconv_x3_pack_weight(pdev(model, u.pw), u.cout, u.k, u.cin, u.scale, u.packed.ptr, st,
                             u.arith);
        continue;
      }
      const int64_t n = tconv_packed_floats(u.cout, u.k, u.cin);
      u.packed.ensure((size_t)n * sizeof(float));
      tconv_pack_weight(pdev(model, u.pw), u.cout, u.k, u.cin, u.packed.as<float>(), st);
    }
    hip_check(hipStreamSynchronize(st), "weight packing");
    model->finalize_failed = false;
    model->finalized = true;
  });
}

int nnx_model_share_workspace(nnx_model* model, nnx_model* owner) {
  return guarded([&] {
    require(model && owner, "null argument");
    if (!owner->ws) owner->ws = std::make_shared<Workspace>();
    model->ws = owner->ws;
  });
}

int nnx_set_layer_checks(int enable) {
  return guarded([&] { g_layer_checks.store(enable != 0, std::memory_order_relaxed); });
}

int nnx_forward(nnx_model* model, const float* d_in, float* d_out, int n, const int* spatial,
                void* stream) {
  return guarded([&] {
    require(spatial != nullptr, "spatial must not be null");
    run_forward(model, d_in, d_out, n, spatial, as_stream(stream));
  });
}

void nnx_model_destroy(nnx_model* model) { delete model; }

int nnx_sw_predict(nnx_model* const* folds, int nfolds, const nnx_sw_config* config,
                   const float* d_volume, void* d_logits, uint16_t* d_labels, void* stream) {
  return guarded([&] {
    require(folds != nullptr && nfolds >= 1, "fold inference requires at least one model");
    validate_sw(config);
    std::vector<nnx_forward_fn> fns(nfolds, &ModelForward::call);
    std::vector<void*> users(nfolds);
    for (int f = 0; f < nfolds; ++f) {
      require(folds[f] != nullptr, "fold model must not be null");
      require(folds[f]->finalized, "fold model is not finalized");
      require(folds[f]->cin == config->channels, "model input channels do not match the volume");
      require(folds[f]->classes == config->num_classes, "model classes do not match");
      users[f] = folds[f];
    }
    sw_run(fns.data(), users.data(), nfolds, config, d_volume, d_logits, d_labels,
           as_stream(stream));
  });
}

int nnx_sw_predict_custom(nnx_forward_fn const* forwards, void* const* users, int nfolds,
                          const nnx_sw_config* config, const float* d_volume, void* d_logits,
                          uint16_t* d_labels, void* stream) {
  return guarded([&] {
    require(forwards && users, "null argument");
    sw_run(forwards, users, nfolds, config, d_volume, d_logits, d_labels, as_stream(stream));
  });
}

void nnx_sw_release(void) {
  SwCache& c = sw_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  c.acc.release();
  c.norm.release();
  c.total.release();
  c.batch_in.release();
  c.batch_out.release();
  c.counter.release();
}

int nnx_count_nonfinite(const float* d_x, int64_t n, unsigned int* d_count, void* stream) {
  return guarded([&] { count_nonfinite(d_x, n, d_count, as_stream(stream)); });
}

size_t nnx_instnorm_workspace_bytes(int batch, int64_t spatial, int channels) {
  try {
    return instnorm_workspace_bytes(batch, spatial, channels);
  } catch (...) {
    return 0;
  }
}

int nnx_instnorm_lrelu(const float* d_x, float* d_y, int batch, int64_t spatial, int channels,
                       const float* d_input_bias, const float* d_gamma, const float* d_beta,
                       float eps, int apply_act, float slope, const float* d_residual,
                       void* d_workspace, size_t workspace_bytes, void* stream) {
  return guarded([&] {
    instnorm_lrelu(d_x, d_y, batch, spatial, channels, d_input_bias, d_gamma, d_beta, eps,
                   apply_act != 0, slope, d_residual, d_workspace, workspace_bytes,
                   as_stream(stream));
  });
}

size_t nnx_instnorm_noalloc_max_bytes(void) { return instnorm_noalloc_max_bytes(); }

int nnx_instnorm_lrelu_noalloc(const float* d_x, float* d_y, int batch, int64_t spatial,
                               int channels, const float* d_input_bias, const float* d_gamma,
                               const float* d_beta, float eps, int apply_act, float slope,
                               const float* d_residual, void* stream) {
  return guarded([&] {
    instnorm_lrelu_noalloc(d_x, d_y, batch, spatial, channels, d_input_bias, d_gamma, d_beta,
                           eps, apply_act != 0, slope, d_residual, as_stream(stream));
  });
}

size_t nnx_conv3d_packed_floats(int cout, const int* ksize, int c1, int c2) {
  if (!ksize || cout < 1 || c1 < 1 || c2 < 0) return 0;
  return (size_t)conv_packed_floats(cout, ksize, c1, c2);
}

int nnx_conv3d_pack_weight(const float* d_weight, int cout, const int* ksize, int c1, int c2,
                           float* d_packed, void* stream) {
  return guarded([&] {
    require(d_weight && ksize && d_packed, "null argument");
    conv_pack_weight(d_weight, cout, ksize, c1, c2, d_packed, as_stream(stream));
  });
}

int nnx_conv3d_igemm(const float* d_x1, int c1, const float* d_x2, int c2,
                     const float* d_packed, const float* d_bias, float* d_y, int batch,
                     const int* in_size, int cout, const int* ksize, const int* stride,
                     void* stream) {
  return guarded([&] {
    require(in_size && ksize && stride, "null argument");
    require(cout >= 1, "convolution needs at least one output channel");
    const ConvGeom g = make_conv_geom(batch, in_size, ksize, stride);
    conv3d_igemm(d_x1, c1, d_x2, c2, d_packed, d_bias, d_y, g, cout, as_stream(stream));
  });
}

float nnx_split_weight_scale(float max_abs) {
  if (!(max_abs >= 0.f) || !std::isfinite(max_abs)) return 0.f;
  return split_weight_scale(max_abs);
}

size_t nnx_conv3d_split_packed_bytes(int cout, const int* ksize, int c1, int c2) {
  if (!ksize || cout < 1 || c1 < 1 || c2 < 0) return 0;
  return (size_t)conv_x3_packed_bytes(cout, ksize, c1, c2);
}

int nnx_conv3d_split_pack_weight(const float* d_weight, int cout, const int* ksize, int c1,
                                 int c2, float scale, void* d_packed, void* stream) {
  return guarded([&] {
    require(d_weight && ksize && d_packed, "null argument");
    conv_x3_pack_weight(d_weight, cout, ksize, c1, c2, scale, d_packed, as_stream(stream));
  });
}

int nnx_conv3d_split(const float* d_x1, int c1, const float* d_x2, int c2, const void* d_packed,
                     float scale, const float* d_bias, float* d_y, int batch, const int* in_size,
                     int cout, const int* ksize, const int* stride, void* stream) {
  return guarded([&] {
    require(in_size && ksize && stride, "null argument");
    require(cout >= 1, "convolution needs at least one output channel");
    const ConvGeom g = make_conv_geom(batch, in_size, ksize, stride);
    conv3d_x3(d_x1, c1, d_x2, c2, d_packed, scale, d_bias, d_y, g, cout, as_stream(stream));
  });
}

float nnx_winograd_weight_scale(float max_abs) {
  if (!(max_abs >= 0.f) || !std::isfinite(max_abs)) return 0.f;
  return wino_weight_scale(max_abs);
}

size_t nnx_conv3d_winograd_packed_bytes(int cout, int c1, int c2) {
  if (cout < 1 || c1 < 1 || c2 < 0) return 0;
  return (size_t)conv_wino_packed_bytes(cout, c1, c2);
}

int nnx_conv3d_winograd_pack_weight(const float* d_weight, int cout, int c1, int c2, float scale,
                                    void* d_packed, void* stream) {
  return guarded([&] {
    conv_wino_pack_weight(d_weight, cout, c1, c2, scale, d_packed, as_stream(stream));
  });
}

int nnx_conv3d_winograd(const float* d_x1, int c1, const float* d_x2, int c2, const void* d_packed,
                        float scale, const float* d_bias, float* d_y, int batch,
                        const int* in_size, int cout, void* stream) {
  return guarded([&] {
    require(in_size != nullptr, "null argument");
    const int k3[3] = {3, 3, 3}, s1[3] = {1, 1, 1};
    const ConvGeom g = make_conv_geom(batch, in_size, k3, s1);
    conv3d_wino(d_x1, c1, d_x2, c2, d_packed, scale, d_bias, d_y, g, cout, as_stream(stream));
  });
}

int nnx_conv3d_direct_small_cin(const float* d_x, const float* d_weight, const float* d_bias,
                                float* d_y, int batch, const int* size, int cout, void* stream) {
  return guarded([&] {
    require(size != nullptr, "null argument");
    conv3d_direct_cin1(d_x, d_weight, d_bias, d_y, batch, size, cout, as_stream(stream));
  });
}

int nnx_conv3d_direct_small_cin_split(const float* d_x, int cin, const float* d_weight,
                                      float scale, const float* d_bias, float* d_y, int batch,
                                      const int* size, int cout, void* stream) {
  return guarded([&] {
    require(size != nullptr, "null argument");
    require(cin == 1 || cin == 2 || cin == 4,
            "the split direct convolution takes 1, 2 or 4 input channels");
    require(scale > 0.f && std::isfinite(scale), "weight scale must be positive");
    conv3d_direct_cin1(d_x, d_weight, d_bias, d_y, batch, size, cout, as_stream(stream), nullptr,
                       scale, cin);
  });
}

size_t nnx_tconv3d_packed_floats(int cout, const int* ksize, int cin) {
  if (!ksize || cout < 1 || cin < 1) return 0;
  return (size_t)tconv_packed_floats(cout, ksize, cin);
}

int nnx_tconv3d_pack_weight(const float* d_weight, int cout, const int* ksize, int cin,
                            float* d_packed, void* stream) {
  return guarded([&] {
    require(d_weight && ksize && d_packed, "null argument");
    tconv_pack_weight(d_weight, cout, ksize, cin, d_packed, as_stream(stream));
  });
}

int nnx_tconv3d_gemm(const float* d_x, int cin, const float* d_packed, const float* d_bias,
                     float* d_y, int batch, const int* in_size, int cout, const int* ksize,
                     void* stream) {
  return guarded([&] {
    require(in_size && ksize, "null argument");
    require(batch >= 1 && cout >= 1, "invalid transposed-convolution sizes");
    tconv3d_gemm(d_x, cin, d_packed, d_bias, d_y, batch, in_size, cout, ksize, as_stream(stream));
  });
}

size_t nnx_tconv3d_split_packed_bytes(int cout, const int* ksize, int cin) {
  if (!ksize || cout < 1 || cin < 1) return 0;
  return (size_t)tconv_x3_packed_bytes(cout, ksize, cin);
}

int nnx_tconv3d_split_pack_weight(const float* d_weight, int cout, const int* ksize, int cin,
                                  float scale, void* d_packed, void* stream) {
  return guarded([&] {
    require(d_weight && ksize && d_packed, "null argument");
    tconv_x3_pack_weight(d_weight, cout, ksize, cin, scale, d_packed, as_stream(stream));
  });
}

int nnx_tconv3d_split(const float* d_x, int cin, const void* d_packed, float scale,
                      const float* d_bias, float* d_y, int batch, const int* in_size, int cout,
                      const int* ksize, void* stream) {
  return guarded([&] {
    require(in_size && ksize, "null argument");
    require(batch >= 1 && cout >= 1, "invalid transposed-convolution sizes");
    tconv3d_x3(d_x, cin, d_packed, scale, d_bias, d_y, batch, in_size, cout, ksize,
               as_stream(stream));
  });
}

int nnx_conv3d_bf16_pack_weight(const float* d_weight, int cout, const int* ksize, int c1, int c2,
                                float scale, void* d_packed, void* stream) {
  return guarded([&] {
    require(d_weight && ksize && d_packed, "null argument");
    conv_x3_pack_weight(d_weight, cout, ksize, c1, c2, scale, d_packed, as_stream(stream),
                        kArithBf16);
  });
}

int nnx_conv3d_bf16(const float* d_x1, int c1, const float* d_x2, int c2, const void* d_packed,
                    float scale, const float* d_bias, float* d_y, int batch, const int* in_size,
                    int cout, const int* ksize, const int* stride, void* stream) {
  return guarded([&] {
    require(in_size && ksize && stride, "null argument");
    require(cout >= 1, "convolution needs at least one output channel");
    const ConvGeom g = make_conv_geom(batch, in_size, ksize, stride);
    conv3d_x3(d_x1, c1, d_x2, c2, d_packed, scale, d_bias, d_y, g, cout, as_stream(stream),
              nullptr, {}, {}, kArithBf16);
  });
}

int nnx_tconv3d_bf16_pack_weight(const float* d_weight, int cout, const int* ksize, int cin,
                                 float scale, void* d_packed, void* stream) {
  return guarded([&] {
    require(d_weight && ksize && d_packed, "null argument");
    tconv_x3_pack_weight(d_weight, cout, ksize, cin, scale, d_packed, as_stream(stream),
                         kArithBf16);
  });
}

int nnx_tconv3d_bf16(const float* d_x, int cin, const void* d_packed, float scale,
                     const float* d_bias, float* d_y, int batch, const int* in_size, int cout,
                     const int* ksize, void* stream) {
  return guarded([&] {
    require(in_size && ksize, "null argument");
    require(batch >= 1 && cout >= 1, "invalid transposed-convolution sizes");
    tconv3d_x3(d_x, cin, d_packed, scale, d_bias, d_y, batch, in_size, cout, ksize,
               as_stream(stream), kArithBf16);
  });
}

int nnx_restore_labels(const void* d_logits, int half, int classes, const int* src_shape,
                       const int* dst_shape, uint16_t* d_labels, void* stream) {
  return guarded([&] {
    require(src_shape && dst_shape, "null argument");
    restore_labels(d_logits, half != 0, classes, src_shape, dst_shape, d_labels,
                   as_stream(stream));
  });
}

size_t nnx_restore_labels_spline_workspace(const int* src_shape, const int* dst_shape,
                                           int separate_axis) {
  if (!src_shape || !dst_shape || separate_axis < -1 || separate_axis > 2) return 0;
  for (int a = 0; a < 3; ++a)
    if (src_shape[a] < 1 || dst_shape[a] < 1) return 0;
  return restore_labels_spline_workspace(src_shape, dst_shape, separate_axis);
}

int nnx_restore_labels_spline(const void* d_logits, int half, int classes, const int* src_shape,
                              const int* dst_shape, int order, int separate_axis, void* d_work,
                              size_t work_bytes, uint16_t* d_labels, void* stream) {
  return guarded([&] {
    require(src_shape && dst_shape, "null argument");
    restore_labels_spline(d_logits, half != 0, classes, src_shape, dst_shape, order,
                          separate_axis, d_work, work_bytes, d_labels, as_stream(stream));
  });
}

int nnx_torch_resize(const void* d_in, int half, int channels, const int* in_size,
                     const int64_t* in_strides, float* d_out, const int* out_size,
                     const int64_t* out_strides, int mode, void* stream) {
  return guarded([&] {
    torch_resize(d_in, half != 0, channels, in_size, in_strides, d_out, out_size, out_strides,
                 mode, as_stream(stream));
  });
}

int nnx_torch_resize_argmax(const void* d_logits, int half, int classes, const int* in_size,
                            const int64_t* in_strides, const int* out_size, int mode,
                            uint16_t* d_labels, void* stream) {
  return guarded([&] {
    torch_resize_argmax(d_logits, half != 0, classes, in_size, in_strides, out_size, mode,
                        d_labels, as_stream(stream));
  });
}

int nnx_nonzero_bbox(const float* d_data, int channels, const int64_t* size, int* d_bbox,
                     void* stream) {
  return guarded([&] { nonzero_bbox(d_data, channels, size, d_bbox, as_stream(stream)); });
}

int nnx_crop_normalize(const float* d_data, int channels, const int64_t* size,
                       const int* transpose, const int64_t* start, const int64_t* out_size,
                       const int* schemes, const float* norm, float* d_out, void* stream) {
  return guarded([&] {
    crop_normalize(d_data, channels, size, transpose, start, out_size, schemes, norm, d_out,
                   as_stream(stream));
  });
}

int nnx_nonzero_mask_filled(const float* d_data, int channels, const int64_t* size,
                            const int64_t* start, const int64_t* extent, uint8_t* d_mask,
                            void* d_work, void* stream) {
  int rounds = 0;
  const int rc = guarded([&] {
    rounds = nonzero_mask_filled(d_data, channels, size, start, extent, d_mask, d_work,
                                 as_stream(stream));
  });
  return rc != 0 ? rc : rounds;
}

size_t nnx_zscore_stats_workspace(void) { return zscore_stats_workspace(); }

int nnx_channel_minmax(const float* d_data, int channels, const int64_t* size, int channel,
                       const int64_t* start, const int64_t* extent, float* d_minmax,
                       void* d_work, void* stream) {
  return guarded([&] {
    box_minmax(d_data, channels, size, channel, start, extent, d_minmax, d_work,
               as_stream(stream));
  });
}

int nnx_zscore_stats(const float* d_data, int channels, const int64_t* size, int channel,
                     const int64_t* start, const int64_t* extent, const uint8_t* d_mask,
                     float* d_stats, void* d_work, void* stream) {
  return guarded([&] {
    zscore_stats(d_data, channels, size, channel, start, extent, d_mask, d_stats, d_work,
                 as_stream(stream));
  });
}

int nnx_crop_normalize_masked(const float* d_data, int channels, const int64_t* size,
                              const int* transpose, const int64_t* start,
                              const int64_t* out_size, const int* schemes, const float* norm,
                              const uint8_t* d_mask, const int64_t* mask_start,
                              const int64_t* mask_extent, float* d_out, void* stream) {
  return guarded([&] {
    crop_normalize_masked(d_data, channels, size, transpose, start, out_size, schemes, norm,
                          d_mask, mask_start, mask_extent, d_out, as_stream(stream));
  });
}

size_t nnx_resample_spline_workspace(const int64_t* size, const int64_t* new_size,
                                     int separate_axis) {
  if (!size || !new_size || separate_axis < -1 || separate_axis > 2) return 0;
  for (int a = 0; a < 3; ++a)
    if (size[a] < 1 || new_size[a] < 1) return 0;
  return resample_spline_workspace(size, new_size, separate_axis);
}

int nnx_resample_spline(const float* d_data, int channels, const int64_t* size,
                        const int64_t* new_size, int order, int separate_axis, int order_z,
                        void* d_work, size_t work_bytes, float* d_out, void* stream) {
  return guarded([&] {
    resample_spline(d_data, channels, size, new_size, order, separate_axis, order_z, d_work,
                    work_bytes, d_out, as_stream(stream));
  });
}

int nnx_conv1x1(const float* d_x, int cin, const float* d_weight, const float* d_bias, float* d_y,
                int64_t voxels, int cout, void* stream) {
  return guarded([&] { conv1x1(d_x, cin, d_weight, d_bias, d_y, voxels, cout, as_stream(stream)); });
}

int nnx_sw_gather_flip(const float* d_volume, int channels, const int64_t* size,
                       const int* pad_before, const int* offset, const int* patch,
                       const int* view_flips, int nviews, float* d_out, void* stream) {
  return guarded([&] {
    require(size && pad_before && offset && patch && view_flips, "null argument");
    sw_gather_flip(d_volume, channels, size, pad_before, offset, patch, view_flips, nviews, d_out,
                   as_stream(stream));
  });
}

int nnx_sw_accumulate(const float* d_pred, int nviews, const int* view_flips, int num_classes,
                      const int* patch, const void* d_gaussian, const int* offset,
                      const int64_t* padded, int accumulation, void* d_acc, void* d_norm,
                      void* stream) {
  return guarded([&] {
    require(view_flips && patch && offset && padded, "null argument");
    require(accumulation == NNX_ACCUM_F32 || accumulation == NNX_ACCUM_NNUNET_F16,
            "unsupported sliding-window accumulation");
    sw_accumulate(d_pred, nviews, view_flips, num_classes, patch, d_gaussian, offset, padded,
                  accumulation, d_acc, d_norm, as_stream(stream));
  });
}

int nnx_sw_fold_add(const void* d_acc, const void* d_norm, int num_classes, const int64_t* padded,
                    const int* crop_lo, const int64_t* crop_size, int accumulation, int first,
                    void* d_total, void* stream) {
  return guarded([&] {
    require(padded && crop_lo && crop_size, "null argument");
    require(accumulation == NNX_ACCUM_F32 || accumulation == NNX_ACCUM_NNUNET_F16,
            "unsupported sliding-window accumulation");
    sw_fold_add(d_acc, d_norm, num_classes, padded, crop_lo, crop_size, accumulation, first != 0,
                d_total, as_stream(stream));
  });
}

int nnx_sw_fold_finalize(const void* d_total, int num_classes, int64_t voxels, int nfolds,
                         int accumulation, void* d_logits, uint16_t* d_labels,
                         unsigned int* d_invalid, void* stream) {
  return guarded([&] {
    require(accumulation == NNX_ACCUM_F32 || accumulation == NNX_ACCUM_NNUNET_F16,
            "unsupported sliding-window accumulation");
    sw_fold_finalize(d_total, num_classes, voxels, nfolds, accumulation, d_logits, d_labels,
                     d_invalid, as_stream(stream));
  });
}

int nnx_profile_begin(void) {
  return guarded([&] {
    ProfState& p = prof_state();
    std::lock_guard<std::mutex> lock(p.mu);
    require(!p.on, "profiling already active");
    p.records.clear();
    p.totals.clear();
    p.on = true;
  });
}

int nnx_profile_end(int* count) {
  return guarded([&] {
    ProfState& p = prof_state();
    std::lock_guard<std::mutex> lock(p.mu);
    require(p.on, "profiling is not active");
    p.on = false;
    std::map<std::string, size_t> slot;
    for (const ProfRecord& r : p.records) {
      hip_check(hipEventSynchronize(r.stop), "hipEventSynchronize");
      float ms = 0.f;
      hip_check(hipEventElapsedTime(&ms, r.start, r.stop), "hipEventElapsedTime");
      auto it = slot.find(r.name);
      if (it == slot.end()) {
        it = slot.emplace(r.name, p.totals.size()).first;
        p.totals.push_back(ProfTotal{r.name});
      }
      ProfTotal& t = p.totals[it->second];
      t.launches += 1;
      t.ms += ms;
      t.flops += r.flops;
      t.bytes += r.bytes;
      p.pool.push_back(r.start);
      p.pool.push_back(r.stop);
    }
    p.records.clear();
    if (count) *count = (int)p.totals.size();
  });
}

int nnx_profile_read(int index, const char** name, int* launches, double* milliseconds,
                     double* flops, double* bytes) {
  return guarded([&] {
    ProfState& p = prof_state();
    std::lock_guard<std::mutex> lock(p.mu);
    require(index >= 0 && index < (int)p.totals.size(), "profile index out of range");
    const ProfTotal& t = p.totals[index];
    if (name) *name = t.name.c_str();
    if (launches) *launches = t.launches;
    if (milliseconds) *milliseconds = t.ms;
    if (flops) *flops = t.flops;
    if (bytes) *bytes = t.bytes;
  });
}

int nnx_avgpool3d(const float* d_x, float* d_y, int batch, const int* in_size, int channels,
                  const int* kernel, void* stream) {
  return guarded([&] {
    require(in_size && kernel, "null argument");
    avgpool3d(d_x, d_y, batch, in_size, channels, kernel, as_stream(stream));
  });
}

}  // extern "C"
