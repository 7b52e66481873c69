// extern "C" entry points of libmiq_qconv: host-side validation, kernel selection and
// error reporting.  No entry point touches the GPU before its arguments are validated.  The
// only one that allocates device memory is miq_grad_nhwc_f32 (its ordered split sums keep a
// grow-only workspace per device, as the reference's launch_grad_nhwc does).

#include <cmath>
#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "grow_buffer.h"
#include "miq_qconv.h"
#include "qconv_internal.h"

namespace {

thread_local std::string g_last_error;

int fail(int status, const std::string& msg) {
  g_last_error = msg;
  return status;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(MIQ_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

constexpr long long kMaxDirectElems = 0xFFFFFF00LL;  // one thread per output element, 32-bit grid

// Output geometry with the checks, order and messages of infer_conv_shape
// (/root/reference/src/conv_types.h:125-146).  The filter's cin_per_group is c / groups by
// construction on this interface (as in cuda_kernels.cu:1341-1343), so the reference's
// "filter cin_per_group mismatch" cannot arise.  Negative extents, which the reference
// would pass to std::vector, are rejected here; intermediate sums use 64-bit arithmetic.
int infer_geom(int32_t n, int32_t h, int32_t w, int32_t c, int32_t r, int32_t s, int32_t k,
               const miq_conv2d_params* p, miq::Geom* g) {
  if (p == nullptr) return fail(MIQ_ERR_NULL_POINTER, "convolution parameters pointer is NULL");
  if (n < 0 || h < 0 || w < 0 || c < 0 || r < 0 || s < 0 || k < 0) {
    return fail(MIQ_ERR_INVALID_ARGUMENT, "tensor extents must be >= 0");
  }
  if (p->groups <= 0) return fail(MIQ_ERR_INVALID_ARGUMENT, "groups must be > 0");
  if (c % p->groups != 0) return fail(MIQ_ERR_INVALID_ARGUMENT, "input channels must be divisible by groups");
  if (k % p->groups != 0) return fail(MIQ_ERR_INVALID_ARGUMENT, "output channels must be divisible by groups");
  const long long rows = static_cast<long long>(h) + 2LL * p->pad_h - static_cast<long long>(p->dilation_h) * (r - 1) - 1;
  const long long cols = static_cast<long long>(w) + 2LL * p->pad_w - static_cast<long long>(p->dilation_w) * (s - 1) - 1;
  if (rows < 0 || cols < 0) return fail(MIQ_ERR_INVALID_ARGUMENT, "invalid output size (negative numerator)");
  if (p->stride_h <= 0 || p->stride_w <= 0) return fail(MIQ_ERR_INVALID_ARGUMENT, "stride must be > 0");
  const long long ho = rows / p->stride_h + 1;
  const long long wo = cols / p->stride_w + 1;
  if (ho <= 0 || wo <= 0) return fail(MIQ_ERR_INVALID_ARGUMENT, "computed output size is <= 0");
  if (ho > 0x7fffffffLL || wo > 0x7fffffffLL) return fail(MIQ_ERR_INVALID_ARGUMENT, "output size overflows int32");
  g->N = n; g->H = h; g->W = w; g->C = c;
  g->K = k; g->R = r; g->S = s;
  g->Ho = static_cast<int>(ho); g->Wo = static_cast<int>(wo);
  g->ph = p->pad_h; g->pw = p->pad_w;
  g->sh = p->stride_h; g->sw = p->stride_w;
  g->dh = p->dilation_h; g->dw = p->dilation_w;
  g->G = p->groups; g->Cg = c / p->groups; g->Kg = k / p->groups;
  return MIQ_OK;
}

// Blocked geometry with the rules of infer_block_conv_shape (conv_types.h:148-169).
int infer_block_geom(int32_t n, int32_t h, int32_t w, int32_t c, int32_t r, int32_t s, int32_t k,
                     const miq_block_conv2d_params* p, miq::Geom* g, miq::BlockGeom* bg) {
  if (p == nullptr) return fail(MIQ_ERR_NULL_POINTER, "blocked convolution parameters pointer is NULL");
  if (p->block_by <= 0 || p->block_bx <= 0) return fail(MIQ_ERR_INVALID_ARGUMENT, "block_by and block_bx must be > 0");
  const int st = infer_geom(n, h, w, c, r, s, k, &p->conv, g);
  if (st != MIQ_OK) return st;
  if (g->Ho % p->block_by != 0 || g->Wo % p->block_bx != 0) {
    return fail(MIQ_ERR_INVALID_ARGUMENT, "blocked convolution requires Ho/Wo divisible by block grid");
  }
  bg->By = p->block_by; bg->Bx = p->block_bx;
  bg->bho = g->Ho / p->block_by; bg->bwo = g->Wo / p->block_bx;
  return MIQ_OK;
}

long long out_elems(const miq::Geom& g) { return static_cast<long long>(g.N) * g.Ho * g.Wo * g.K; }
long long in_elems(const miq::Geom& g) { return static_cast<long long>(g.N) * g.H * g.W * g.C; }
long long filt_elems(const miq::Geom& g) { return static_cast<long long>(g.K) * g.R * g.S * g.Cg; }

int check_tensors(const miq::Geom& g, long long filt, const void* x, const void* w, const void* y) {
  if (out_elems(g) > 0 && y == nullptr) return fail(MIQ_ERR_NULL_POINTER, "output pointer is NULL");
  if (in_elems(g) > 0 && x == nullptr) return fail(MIQ_ERR_NULL_POINTER, "input pointer is NULL");
  if (filt > 0 && w == nullptr) return fail(MIQ_ERR_NULL_POINTER, "filter pointer is NULL");
  if (out_elems(g) > kMaxDirectElems) return fail(MIQ_ERR_UNSUPPORTED, "output has more than 2^32-256 elements");
  return MIQ_OK;
}

// The fp32 forward pass (miq_fprop_nhwc_f32, miq_block_fprop_nhwc_f32): bias and the
// depthwise kernel only with a plain filter and no bias.
int fprop_f32(const miq::Geom& g, const miq::BlockGeom& bg, const float* x, const float* w, const float* bias,
              int32_t bias_mode, float* y, int32_t algo, void* stream) {
  int st = check_tensors(g, filt_elems(g) * bg.By * bg.Bx, x, w, y);
  if (st != MIQ_OK) return st;
  if (bias_mode != 0 && bias_mode != 1) return fail(MIQ_ERR_INVALID_ARGUMENT, "bias_mode must be 0 (per block) or 1 (shared)");
  std::string why;
  bool igemm = false;
  switch (algo) {
    case MIQ_ALGO_AUTO: igemm = miq::f32_igemm_eligible(g, bg, x, w, nullptr); break;
    case MIQ_ALGO_DIRECT: igemm = false; break;
    case MIQ_ALGO_IGEMM:
      if (!miq::f32_igemm_eligible(g, bg, x, w, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      igemm = true;
      break;
    default: return fail(MIQ_ERR_INVALID_ARGUMENT, "fp32 convolution algo must be AUTO, DIRECT or IGEMM");
  }
  if (out_elems(g) == 0) return MIQ_OK;
  const hipStream_t hs = static_cast<hipStream_t>(stream);
  const bool dense = bg.By == 1 && bg.Bx == 1 && bias == nullptr;
  hipError_t e;
  if (igemm) {
    e = miq::launch_f32_igemm(g, bg, x, w, bias, bias_mode, y, hs);
  } else if (algo == MIQ_ALGO_AUTO && dense && miq::f32_depthwise_eligible(g, x, y)) {
    e = miq::launch_f32_depthwise(g, x, w, y, hs);
  } else {
    e = miq::launch_f32_direct(g, bg, x, w, bias, bias_mode, y, hs);
  }
  if (e != hipSuccess) return hip_fail(e, "fp32 convolution launch");
  return MIQ_OK;
}

// The fp32 dx pass (miq_bprop_nhwc_f32, miq_block_bprop_nhwc_f32).
int bprop_f32(const miq::Geom& g, const miq::BlockGeom& bg, const float* dy, const float* w, float* dx, int32_t algo,
              void* stream) {
  // dy has the output's extent, dx the input's
  if (in_elems(g) > 0 && dx == nullptr) return fail(MIQ_ERR_NULL_POINTER, "dx pointer is NULL");
  if (out_elems(g) > 0 && dy == nullptr) return fail(MIQ_ERR_NULL_POINTER, "dy pointer is NULL");
  if (filt_elems(g) * bg.By * bg.Bx > 0 && w == nullptr) return fail(MIQ_ERR_NULL_POINTER, "filter pointer is NULL");
  if (in_elems(g) > kMaxDirectElems) return fail(MIQ_ERR_UNSUPPORTED, "dx has more than 2^32-256 elements");
  std::string why;
  bool igemm = false;
  switch (algo) {
    case MIQ_ALGO_AUTO: igemm = miq::f32_bprop_igemm_eligible(g, bg, dy, w, nullptr); break;
    case MIQ_ALGO_DIRECT: igemm = false; break;
    case MIQ_ALGO_IGEMM:
      if (!miq::f32_bprop_igemm_eligible(g, bg, dy, w, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      igemm = true;
      break;
    default: return fail(MIQ_ERR_INVALID_ARGUMENT, "fp32 bprop algo must be AUTO, DIRECT or IGEMM");
  }
  if (in_elems(g) == 0) return MIQ_OK;
  const hipStream_t hs = static_cast<hipStream_t>(stream);
  const bool dense = bg.By == 1 && bg.Bx == 1;
  const hipError_t e = igemm ? miq::launch_f32_bprop_igemm(g, bg, dy, w, dx, hs)
                       : algo == MIQ_ALGO_AUTO && dense && miq::f32_depthwise_bprop_eligible(g, dy, dx)
                           ? miq::launch_f32_depthwise_bprop(g, dy, w, dx, hs)
                           : miq::launch_f32_bprop_direct(g, bg, dy, w, dx, hs);
  if (e != hipSuccess) return hip_fail(e, "fp32 bprop launch");
  return MIQ_OK;
}

// hipMalloc as grow_buffer's allocator: 0 or the HIP error (cleared from the thread's last
// error, so a failed doubled request does not surface in a later call).
struct HipAlloc {
  hipError_t err = hipSuccess;
  int operator()(void** p, size_t bytes) {
    err = hipMalloc(p, bytes);
    if (err != hipSuccess) {
      (void)hipGetLastError();
      *p = nullptr;
      return 1;
    }
    return 0;
  }
};

// The float-code row-band and stream paths' workspace (the prepass's output) behind the
// reference-signature entry points: one grow-only buffer per (device, stream), at most
// kMaxQi32Workspaces of them.  Calls on one stream are ordered and share it; calls on
// different streams never share one.  Neither growth nor any other call here synchronises.
struct StreamKey {
  int dev;
  hipStream_t stream;
  bool operator==(const StreamKey& o) const { return dev == o.dev && stream == o.stream; }
};
constexpr size_t kMaxQi32Workspaces = 64;
std::mutex g_qi32_ws_m;
miq::GrowBufferTable<StreamKey> g_qi32_ws(kMaxQi32Workspaces);

int stream_workspace(hipStream_t s, size_t bytes, void** out) {
  *out = nullptr;
  if (bytes == 0) return MIQ_OK;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_qi32_ws_m);
  miq::GrowBuffer* b = g_qi32_ws.find_or_add(StreamKey{dev, s});
  if (b == nullptr) {
    return fail(MIQ_ERR_UNSUPPORTED,
                "the float-code workspace table is full (64 (device, stream) pairs); use miq_fprop_nhwc_qi32_ws");
  }
  HipAlloc alloc;
  if (miq::grow_buffer(*b, bytes, alloc, out) != 0) return hip_fail(alloc.err, "hipMalloc of the qi32 workspace");
  return MIQ_OK;
}

// Bytes of workspace a float-code problem needs on the kernel `algo` (resolved, not AUTO).
size_t qi32_workspace_bytes(const miq::Geom& g, const miq::BlockGeom& bg, int32_t algo) {
  if (algo == MIQ_ALGO_BAND) return miq::qi32_band_workspace_bytes(g, bg);
  if (algo == MIQ_ALGO_STREAM) return miq::qi32_route_workspace_bytes(g);
  if (algo == MIQ_ALGO_STEM_S2D) return miq::qi32_stem_route_workspace_bytes(g);
  return 0;
}

// The kernel AUTO runs for a float-code problem: the row-band kernel, else the stream route,
// else the stem route, else the implicit GEMM, else the direct kernel.
int32_t qi32_auto(const miq::Geom& g, const miq::BlockGeom& bg, const void* x, const void* w, const void* y) {
  if (miq::qi32_band_eligible(g, bg, x, w, y, nullptr)) return MIQ_ALGO_BAND;
  if (miq::qi32_route_eligible(g, bg, x, w, y, nullptr)) return MIQ_ALGO_STREAM;
  if (miq::qi32_stem_route_eligible(g, bg, x, w, y, nullptr)) return MIQ_ALGO_STEM_S2D;
  if (miq::qi32_igemm_eligible(g, bg, x, w, nullptr)) return MIQ_ALGO_IGEMM;
  return MIQ_ALGO_DIRECT;
}

// A caller workspace for qi32_entry: `given` false means the library's own (stream_workspace).
struct CallerWorkspace {
  bool given = false;
  void* p = nullptr;
  size_t bytes = 0;
};

int qi32_entry(miq::QpKind qk, const float* x, const float* w, int32_t* y, const miq::Geom& g,
               const miq::BlockGeom& bg, const void* in_qp, const void* f_qp, void* stream,
               int32_t algo = MIQ_ALGO_AUTO, CallerWorkspace cw = CallerWorkspace{}) {
  const long long filt = filt_elems(g) * bg.By * bg.Bx;
  int st = check_tensors(g, filt, x, w, y);
  if (st != MIQ_OK) return st;
  if (in_qp == nullptr || f_qp == nullptr) {
    return fail(MIQ_ERR_NULL_POINTER, "quantized fprop requires non-null quantization parameters");
  }
  std::string why;
  switch (algo) {
    case MIQ_ALGO_AUTO: algo = qi32_auto(g, bg, x, w, y); break;
    case MIQ_ALGO_DIRECT: break;
    case MIQ_ALGO_IGEMM:
      if (!miq::qi32_igemm_eligible(g, bg, x, w, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      break;
    case MIQ_ALGO_BAND:
      if (!miq::qi32_band_eligible(g, bg, x, w, y, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      break;
    case MIQ_ALGO_STREAM:
      if (!miq::qi32_route_eligible(g, bg, x, w, y, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      break;
    case MIQ_ALGO_STEM_S2D:
      if (!miq::qi32_stem_route_eligible(g, bg, x, w, y, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      break;
    default:
      return fail(MIQ_ERR_INVALID_ARGUMENT,
                  "float-code convolution algo must be AUTO, DIRECT, IGEMM, BAND, STREAM or STEM_S2D");
  }
  const size_t ws_bytes = qi32_workspace_bytes(g, bg, algo);
  if (cw.given && cw.bytes < ws_bytes) {
    return fail(MIQ_ERR_INVALID_ARGUMENT, "workspace is smaller than miq_fprop_nhwc_qi32_workspace_size reports");
  }
  if (cw.given && ws_bytes > 0 && cw.p == nullptr) return fail(MIQ_ERR_NULL_POINTER, "workspace pointer is NULL");
  if (out_elems(g) == 0) return MIQ_OK;
  const hipStream_t hs = static_cast<hipStream_t>(stream);
  void* ws = cw.p;
  if (!cw.given) {
    st = stream_workspace(hs, ws_bytes, &ws);
    if (st != MIQ_OK) return st;
  }
  hipError_t e;
  switch (algo) {
    case MIQ_ALGO_BAND: {
      e = miq::launch_qi32_band(g, bg, qk, x, w, y, in_qp, f_qp, ws, hs);
      if (e != hipSuccess) return hip_fail(e, "qi32 row-band launch");
      return MIQ_OK;
    }
    case MIQ_ALGO_STREAM: {
      e = miq::launch_qi32_route(g, qk, x, w, y, in_qp, f_qp, ws, hs);
      if (e != hipSuccess) return hip_fail(e, "qi32 stream route launch");
      return MIQ_OK;
    }
    case MIQ_ALGO_STEM_S2D: {
      e = miq::launch_qi32_stem_route(g, qk, x, w, y, in_qp, f_qp, ws, hs);
      if (e != hipSuccess) return hip_fail(e, "qi32 stem route launch");
      return MIQ_OK;
    }
    case MIQ_ALGO_IGEMM:
      e = miq::launch_qi32_igemm(g, bg, qk, x, w, y, in_qp, f_qp, hs);
      if (e != hipSuccess) return hip_fail(e, "qi32 implicit GEMM launch");
      return MIQ_OK;
    default:
      e = miq::launch_qi32_direct(g, bg, qk, x, w, y, in_qp, f_qp, hs);
      if (e != hipSuccess) return hip_fail(e, "qi32 direct convolution launch");
      return MIQ_OK;
  }
}

// Validates an int8 problem and resolves the kernel family.
int plan_i8(const miq_qconv_desc* d, const void* x, const void* w, const void* y, const miq::Requant& rq,
            miq::Epi epi, miq::Geom* g, int32_t* algo) {
  if (d == nullptr) return fail(MIQ_ERR_NULL_POINTER, "descriptor pointer is NULL");
  int st = infer_geom(d->n, d->h, d->w, d->c, d->r, d->s, d->k, &d->conv, g);
  if (st != MIQ_OK) return st;
  std::string why;
  switch (d->algo) {
    case MIQ_ALGO_AUTO:
      if (miq::pointwise_eligible(*g, x, w, y, rq, epi, nullptr)) {
        *algo = MIQ_ALGO_POINTWISE;
      } else if (miq::band_eligible(*g, x, w, y, rq, epi, nullptr)) {
        *algo = MIQ_ALGO_BAND;
      } else if (miq::flat_eligible(*g, x, w, y, rq, epi, nullptr)) {
        *algo = MIQ_ALGO_FLAT;
      } else if (miq::stream_eligible(*g, x, w, y, rq, epi, nullptr)) {
        *algo = MIQ_ALGO_STREAM;
      } else if (miq::dot4_preferred(*g)) {
        *algo = MIQ_ALGO_DOT4;
      } else if (miq::igemm_eligible(*g, x, w, y, epi, nullptr)) {
        *algo = MIQ_ALGO_IGEMM;
      } else if (miq::stem_s2d_eligible(*g, x, w, y, rq, epi, nullptr)) {
        *algo = MIQ_ALGO_STEM_S2D;
      } else if (miq::stem_eligible(*g, x, w, y, epi, nullptr)) {
        *algo = MIQ_ALGO_STEM;
      } else {
        *algo = MIQ_ALGO_DIRECT;
      }
      break;
    case MIQ_ALGO_DIRECT:
      *algo = MIQ_ALGO_DIRECT;
      break;
    case MIQ_ALGO_IGEMM:
      if (!miq::igemm_eligible(*g, x, w, y, epi, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      *algo = MIQ_ALGO_IGEMM;
      break;
    case MIQ_ALGO_STEM:
      if (!miq::stem_eligible(*g, x, w, y, epi, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      *algo = MIQ_ALGO_STEM;
      break;
    case MIQ_ALGO_BAND:
      if (!miq::band_eligible(*g, x, w, y, rq, epi, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      *algo = MIQ_ALGO_BAND;
      break;
    case MIQ_ALGO_STREAM:
      if (!miq::stream_eligible(*g, x, w, y, rq, epi, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      *algo = MIQ_ALGO_STREAM;
      break;
    case MIQ_ALGO_FLAT:
      if (!miq::flat_eligible(*g, x, w, y, rq, epi, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      *algo = MIQ_ALGO_FLAT;
      break;
    case MIQ_ALGO_DOT4:
      if (!miq::dot4_eligible(*g, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      *algo = MIQ_ALGO_DOT4;
      break;
    case MIQ_ALGO_PIPE:
      if (!miq::pipe_eligible(*g, x, w, y, rq, epi, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      *algo = MIQ_ALGO_PIPE;
      break;
    case MIQ_ALGO_POINTWISE:
      if (!miq::pointwise_eligible(*g, x, w, y, rq, epi, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      *algo = MIQ_ALGO_POINTWISE;
      break;
    case MIQ_ALGO_STEM_S2D:
      if (!miq::stem_s2d_eligible(*g, x, w, y, rq, epi, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      *algo = MIQ_ALGO_STEM_S2D;
      break;
    default:
      return fail(MIQ_ERR_INVALID_ARGUMENT, "unknown algo value");
  }
  return MIQ_OK;
}

int i8_entry(miq::Epi epi, const miq_qconv_desc* d, const int8_t* x, const int8_t* w, const int32_t* bias,
             const float* w_scale, void* y, void* stream) {
  miq::Geom g;
  int32_t algo = 0;
  miq::Requant rq{bias, w_scale, 1.0f, d != nullptr && d->relu != 0 ? 1 : 0};
  int st = plan_i8(d, x, w, y, rq, epi, &g, &algo);
  if (st != MIQ_OK) return st;
  st = check_tensors(g, filt_elems(g), x, w, y);
  if (st != MIQ_OK) return st;
  if (epi != miq::kEpiAcc32) {
    if (g.K > 0 && w_scale == nullptr) return fail(MIQ_ERR_NULL_POINTER, "per-channel scale pointer is NULL");
    if (!std::isfinite(d->in_scale) || !std::isfinite(d->out_scale) || d->out_scale == 0.0f) {
      return fail(MIQ_ERR_INVALID_ARGUMENT, "in_scale must be finite and out_scale finite and non-zero");
    }
    rq.act_scale = d->in_scale / d->out_scale;
  }
  if (out_elems(g) == 0) return MIQ_OK;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (algo) {
    case MIQ_ALGO_IGEMM: e = miq::launch_i8_igemm(g, epi, x, w, y, rq, s); break;
    case MIQ_ALGO_STEM: e = miq::launch_i8_stem(g, epi, x, w, y, rq, s); break;
    case MIQ_ALGO_BAND: e = miq::launch_i8_band(g, epi, x, w, y, rq, s); break;
    case MIQ_ALGO_STREAM: e = miq::launch_i8_stream(g, epi, x, w, y, rq, s); break;
    case MIQ_ALGO_FLAT: e = miq::launch_i8_flat(g, epi, x, w, y, rq, s); break;
    case MIQ_ALGO_DOT4: e = miq::launch_i8_dot4(g, epi, x, w, y, rq, s); break;
    case MIQ_ALGO_PIPE: e = miq::launch_i8_pipe(g, epi, x, w, y, rq, s); break;
    case MIQ_ALGO_POINTWISE: e = miq::launch_i8_pointwise(g, x, w, static_cast<int8_t*>(y), rq, s); break;
    case MIQ_ALGO_STEM_S2D: e = miq::launch_i8_stem_s2d(g, x, w, static_cast<int8_t*>(y), rq, s); break;
    default: e = miq::launch_i8_direct(g, epi, x, w, y, rq, s); break;
  }
  if (e != hipSuccess) return hip_fail(e, "int8 convolution launch");
  return MIQ_OK;
}

}  // namespace

extern "C" {

int miq_version(void) { return MIQ_VERSION; }

const char* miq_status_string(int status) {
  switch (status) {
    case MIQ_OK: return "success";
    case MIQ_ERR_NULL_POINTER: return "null pointer argument";
    case MIQ_ERR_INVALID_ARGUMENT: return "invalid argument";
    case MIQ_ERR_UNSUPPORTED: return "unsupported by the requested algorithm";
    case MIQ_ERR_HIP: return "HIP runtime error";
    default: return "unknown status";
  }
}

const char* miq_last_error_message(void) { return g_last_error.c_str(); }

int miq_conv2d_output_shape(int32_t n, int32_t h, int32_t w, int32_t c, int32_t r, int32_t s, int32_t k,
                            const miq_conv2d_params* p, int32_t* ho, int32_t* wo) {
  if (ho == nullptr || wo == nullptr) return fail(MIQ_ERR_NULL_POINTER, "output shape pointer is NULL");
  miq::Geom g;
  const int st = infer_geom(n, h, w, c, r, s, k, p, &g);
  if (st != MIQ_OK) return st;
  *ho = g.Ho;
  *wo = g.Wo;
  return MIQ_OK;
}

int miq_block_conv2d_output_shape(int32_t n, int32_t h, int32_t w, int32_t c, int32_t r, int32_t s, int32_t k,
                                  const miq_block_conv2d_params* p, int32_t* ho, int32_t* wo, int32_t* block_ho,
                                  int32_t* block_wo) {
  if (ho == nullptr || wo == nullptr || block_ho == nullptr || block_wo == nullptr) {
    return fail(MIQ_ERR_NULL_POINTER, "output shape pointer is NULL");
  }
  miq::Geom g;
  miq::BlockGeom bg;
  const int st = infer_block_geom(n, h, w, c, r, s, k, p, &g, &bg);
  if (st != MIQ_OK) return st;
  *ho = g.Ho;
  *wo = g.Wo;
  *block_ho = bg.bho;
  *block_wo = bg.bwo;
  return MIQ_OK;
}

int miq_qconv2d_plan(const miq_qconv_desc* d, int32_t* algo) {
  if (algo == nullptr) return fail(MIQ_ERR_NULL_POINTER, "algo output pointer is NULL");
  miq::Geom g;
  // Alignment is judged for 256-byte aligned allocations (what hipMalloc returns).
  static const char kAligned[16] __attribute__((aligned(256))) = {0};
  const miq::Requant rq{reinterpret_cast<const int32_t*>(kAligned), reinterpret_cast<const float*>(kAligned), 1.0f,
                        d != nullptr && d->relu != 0 ? 1 : 0};
  return plan_i8(d, kAligned, kAligned, kAligned, rq, miq::kEpiI8, &g, algo);
}

int miq_fprop_nhwc_qi32_u8(const float* x, const float* w, int32_t* y, int32_t n, int32_t h, int32_t wdt, int32_t c,
                           int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p, const miq_qparams_u8* in_qp,
                           const miq_qparams_u8* f_qp, void* stream) {
  miq::Geom g;
  const int st = infer_geom(n, h, wdt, c, r, s, k, p, &g);
  if (st != MIQ_OK) return st;
  return qi32_entry(miq::kQpU8, x, w, y, g, miq::BlockGeom{1, 1, g.Ho, g.Wo}, in_qp, f_qp, stream);
}

int miq_fprop_nhwc_qi32_s5(const float* x, const float* w, int32_t* y, int32_t n, int32_t h, int32_t wdt, int32_t c,
                           int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p, const miq_qparams_s5* in_qp,
                           const miq_qparams_s5* f_qp, void* stream) {
  miq::Geom g;
  const int st = infer_geom(n, h, wdt, c, r, s, k, p, &g);
  if (st != MIQ_OK) return st;
  return qi32_entry(miq::kQpS5, x, w, y, g, miq::BlockGeom{1, 1, g.Ho, g.Wo}, in_qp, f_qp, stream);
}

int miq_fprop_nhwc_qi32_algo(int32_t qp_kind, const float* x, const float* w, int32_t* y, int32_t n, int32_t h,
                             int32_t wdt, int32_t c, int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p,
                             const void* in_qp, const void* f_qp, int32_t algo, void* stream) {
  if (qp_kind != 0 && qp_kind != 1) return fail(MIQ_ERR_INVALID_ARGUMENT, "qp_kind must be 0 (LinQuantU8) or 1 (LinQuantS5)");
  miq::Geom g;
  const int st = infer_geom(n, h, wdt, c, r, s, k, p, &g);
  if (st != MIQ_OK) return st;
  return qi32_entry(qp_kind == 0 ? miq::kQpU8 : miq::kQpS5, x, w, y, g, miq::BlockGeom{1, 1, g.Ho, g.Wo}, in_qp, f_qp,
                    stream, algo);
}

int miq_fprop_nhwc_qi32_workspace_size(int32_t n, int32_t h, int32_t wdt, int32_t c, int32_t r, int32_t s,
                                       int32_t k, const miq_conv2d_params* p, int32_t algo, size_t* bytes) {
  if (bytes == nullptr) return fail(MIQ_ERR_NULL_POINTER, "bytes output pointer is NULL");
  *bytes = 0;
  miq::Geom g;
  const int st = infer_geom(n, h, wdt, c, r, s, k, p, &g);
  if (st != MIQ_OK) return st;
  // sized for 256-byte aligned tensors: misaligned ones can only take kernels that need none
  static const char kAligned[16] __attribute__((aligned(256))) = {0};
  const miq::BlockGeom bg{1, 1, g.Ho, g.Wo};
  std::string why;
  switch (algo) {
    case MIQ_ALGO_AUTO: algo = qi32_auto(g, bg, kAligned, kAligned, kAligned); break;
    case MIQ_ALGO_DIRECT:
    case MIQ_ALGO_IGEMM: break;
    case MIQ_ALGO_BAND:
      if (!miq::qi32_band_eligible(g, bg, kAligned, kAligned, kAligned, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      break;
    case MIQ_ALGO_STREAM:
      if (!miq::qi32_route_eligible(g, bg, kAligned, kAligned, kAligned, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      break;
    case MIQ_ALGO_STEM_S2D:
      if (!miq::qi32_stem_route_eligible(g, bg, kAligned, kAligned, kAligned, &why)) {
        return fail(MIQ_ERR_UNSUPPORTED, why);
      }
      break;
    default:
      return fail(MIQ_ERR_INVALID_ARGUMENT,
                  "float-code convolution algo must be AUTO, DIRECT, IGEMM, BAND, STREAM or STEM_S2D");
  }
  *bytes = out_elems(g) == 0 ? 0 : qi32_workspace_bytes(g, bg, algo);
  return MIQ_OK;
}

int miq_fprop_nhwc_qi32_ws(int32_t qp_kind, const float* x, const float* w, int32_t* y, int32_t n, int32_t h,
                           int32_t wdt, int32_t c, int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p,
                           const void* in_qp, const void* f_qp, int32_t algo, void* workspace, size_t workspace_bytes,
                           void* stream) {
  if (qp_kind != 0 && qp_kind != 1) return fail(MIQ_ERR_INVALID_ARGUMENT, "qp_kind must be 0 (LinQuantU8) or 1 (LinQuantS5)");
  miq::Geom g;
  const int st = infer_geom(n, h, wdt, c, r, s, k, p, &g);
  if (st != MIQ_OK) return st;
  CallerWorkspace cw;
  cw.given = true;
  cw.p = workspace;
  cw.bytes = workspace_bytes;
  return qi32_entry(qp_kind == 0 ? miq::kQpU8 : miq::kQpS5, x, w, y, g, miq::BlockGeom{1, 1, g.Ho, g.Wo}, in_qp, f_qp,
                    stream, algo, cw);
}

int miq_plan_block_qi32(int32_t n, int32_t h, int32_t wdt, int32_t c, int32_t r, int32_t s, int32_t k,
                        const miq_block_conv2d_params* p, int32_t* algo) {
  if (algo == nullptr) return fail(MIQ_ERR_NULL_POINTER, "algo output pointer is NULL");
  miq::Geom g;
  miq::BlockGeom bg;
  const int st = infer_block_geom(n, h, wdt, c, r, s, k, p, &g, &bg);
  if (st != MIQ_OK) return st;
  static const char kAligned[16] __attribute__((aligned(256))) = {0};
  *algo = qi32_auto(g, bg, kAligned, kAligned, kAligned);
  return MIQ_OK;
}

int miq_plan_qi32(int32_t n, int32_t h, int32_t wdt, int32_t c, int32_t r, int32_t s, int32_t k,
                  const miq_conv2d_params* p, int32_t* algo) {
  if (algo == nullptr) return fail(MIQ_ERR_NULL_POINTER, "algo output pointer is NULL");
  miq::Geom g;
  const int st = infer_geom(n, h, wdt, c, r, s, k, p, &g);
  if (st != MIQ_OK) return st;
  static const char kAligned[16] __attribute__((aligned(256))) = {0};
  *algo = qi32_auto(g, miq::BlockGeom{1, 1, g.Ho, g.Wo}, kAligned, kAligned, kAligned);
  return MIQ_OK;
}

int miq_block_fprop_nhwc_qi32_u8(const float* x, const float* w, int32_t* y, int32_t n, int32_t h, int32_t wdt,
                                 int32_t c, int32_t r, int32_t s, int32_t k, const miq_block_conv2d_params* p,
                                 const miq_qparams_u8* in_qp, const miq_qparams_u8* f_qp, void* stream) {
  miq::Geom g;
  miq::BlockGeom bg;
  const int st = infer_block_geom(n, h, wdt, c, r, s, k, p, &g, &bg);
  if (st != MIQ_OK) return st;
  return qi32_entry(miq::kQpU8, x, w, y, g, bg, in_qp, f_qp, stream);
}

int miq_block_fprop_nhwc_qi32_s5(const float* x, const float* w, int32_t* y, int32_t n, int32_t h, int32_t wdt,
                                 int32_t c, int32_t r, int32_t s, int32_t k, const miq_block_conv2d_params* p,
                                 const miq_qparams_s5* in_qp, const miq_qparams_s5* f_qp, void* stream) {
  miq::Geom g;
  miq::BlockGeom bg;
  const int st = infer_block_geom(n, h, wdt, c, r, s, k, p, &g, &bg);
  if (st != MIQ_OK) return st;
  return qi32_entry(miq::kQpS5, x, w, y, g, bg, in_qp, f_qp, stream);
}

int miq_qconv2d_nhwc_i8(const miq_qconv_desc* d, const int8_t* x, const int8_t* w, const int32_t* bias,
                        const float* w_scale, int8_t* y, void* stream) {
  return i8_entry(miq::kEpiI8, d, x, w, bias, w_scale, y, stream);
}

int miq_qconv2d_nhwc_i8_acc32(const miq_qconv_desc* d, const int8_t* x, const int8_t* w, int32_t* acc, void* stream) {
  return i8_entry(miq::kEpiAcc32, d, x, w, nullptr, nullptr, acc, stream);
}

int miq_qconv2d_nhwc_i8_dequant(const miq_qconv_desc* d, const int8_t* x, const int8_t* w, const int32_t* bias,
                                const float* w_scale, float* y, void* stream) {
  return i8_entry(miq::kEpiF32, d, x, w, bias, w_scale, y, stream);
}

int miq_fprop_nhwc_f32(const float* x, const float* w, float* y, int32_t n, int32_t h, int32_t wdt, int32_t c,
                       int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p, int32_t algo, void* stream) {
  miq::Geom g;
  const int st = infer_geom(n, h, wdt, c, r, s, k, p, &g);
  if (st != MIQ_OK) return st;
  return fprop_f32(g, miq::dense_blocks(g), x, w, nullptr, 0, y, algo, stream);
}

int miq_block_fprop_nhwc_f32(const float* x, const float* w, float* y, int32_t n, int32_t h, int32_t wdt, int32_t c,
                             int32_t r, int32_t s, int32_t k, const miq_block_conv2d_params* p, const float* bias,
                             int32_t bias_mode, int32_t algo, void* stream) {
  miq::Geom g;
  miq::BlockGeom bg;
  const int st = infer_block_geom(n, h, wdt, c, r, s, k, p, &g, &bg);
  if (st != MIQ_OK) return st;
  return fprop_f32(g, bg, x, w, bias, bias_mode, y, algo, stream);
}

int miq_bprop_nhwc_f32(const float* dy, const float* w, float* dx, int32_t n, int32_t h, int32_t wdt, int32_t c,
                       int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p, int32_t algo, void* stream) {
  miq::Geom g;
  const int st = infer_geom(n, h, wdt, c, r, s, k, p, &g);
  if (st != MIQ_OK) return st;
  return bprop_f32(g, miq::dense_blocks(g), dy, w, dx, algo, stream);
}

int miq_block_bprop_nhwc_f32(const float* dy, const float* w, float* dx, int32_t n, int32_t h, int32_t wdt, int32_t c,
                             int32_t r, int32_t s, int32_t k, const miq_block_conv2d_params* p, int32_t algo,
                             void* stream) {
  miq::Geom g;
  miq::BlockGeom bg;
  const int st = infer_block_geom(n, h, wdt, c, r, s, k, p, &g, &bg);
  if (st != MIQ_OK) return st;
  return bprop_f32(g, bg, dy, w, dx, algo, stream);
}

}  // extern "C"

namespace {

// The kernel family of an fp32 grad call and the workspace bytes of its ordered sums.
enum GradKind { kGradDirect, kGradIgemm, kGradDepthwise };
struct GradChoice {
  GradKind kind;
  bool ordered;      // split sums in a fixed order (workspace); false: float atomics
  size_t ws_bytes;   // dw's split sums, then (with dbias) the bias gradient's runs
  size_t dbias_off;  // byte offset of the bias gradient's runs in the workspace
};

int grad_choose(const miq::Geom& g, const miq::BlockGeom& bg, const void* x, const void* dy, int32_t algo,
                bool with_dbias, GradChoice* ch) {
  std::string why;
  const bool dense = bg.By == 1 && bg.Bx == 1;
  switch (algo) {
    case MIQ_ALGO_AUTO:
    case MIQ_ALGO_ATOMIC:
      ch->kind = dense && miq::f32_depthwise_grad_eligible(g, x, dy) ? kGradDepthwise
                 : miq::f32_grad_igemm_eligible(g, bg, nullptr)      ? kGradIgemm
                                                                     : kGradDirect;
      break;
    case MIQ_ALGO_DIRECT: ch->kind = kGradDirect; break;
    case MIQ_ALGO_IGEMM:
      if (!miq::f32_grad_igemm_eligible(g, bg, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
      ch->kind = kGradIgemm;
      break;
    default: return fail(MIQ_ERR_INVALID_ARGUMENT, "fp32 grad algo must be AUTO, DIRECT, IGEMM or ATOMIC");
  }
  ch->ordered = algo != MIQ_ALGO_ATOMIC;
  const size_t part = !ch->ordered || filt_elems(g) == 0 ? 0
                      : ch->kind == kGradIgemm           ? miq::f32_grad_igemm_workspace(g, bg)
                      : ch->kind == kGradDepthwise       ? miq::f32_depthwise_grad_workspace(g)
                                                         : 0;
  ch->dbias_off = (part + 255) & ~static_cast<size_t>(255);
  ch->ws_bytes = with_dbias ? ch->dbias_off + miq::f32_block_dbias_workspace(g, bg) : part;
  return MIQ_OK;
}

int grad_validate(const float* x, const float* dy, float* dw, const miq::Geom& g, const miq::BlockGeom& bg,
                  const float* dbias, int32_t bias_mode, int32_t algo, GradChoice* ch) {
  const long long filt = filt_elems(g) * bg.By * bg.Bx;
  int st = check_tensors(g, filt, x, dw, dy);
  if (st != MIQ_OK) return st;
  if (filt > kMaxDirectElems) return fail(MIQ_ERR_UNSUPPORTED, "dw has more than 2^32-256 elements");
  if (bias_mode != 0 && bias_mode != 1) return fail(MIQ_ERR_INVALID_ARGUMENT, "bias_mode must be 0 (per block) or 1 (shared)");
  return grad_choose(g, bg, x, dy, algo, dbias != nullptr, ch);
}

int grad_launch(const miq::Geom& g, const miq::BlockGeom& bg, const GradChoice& ch, const float* x, const float* dy,
                float* dw, float* dbias, int32_t bias_mode, void* ws, void* stream) {
  const hipStream_t hs = static_cast<hipStream_t>(stream);
  float* wsf = static_cast<float*>(ws);
  hipError_t e = hipSuccess;
  if (filt_elems(g) > 0) {
    switch (ch.kind) {
      case kGradDepthwise: e = miq::launch_f32_depthwise_grad(g, x, dy, dw, wsf, ch.ordered, hs); break;
      case kGradIgemm: e = miq::launch_f32_grad_igemm(g, bg, x, dy, dw, wsf, ch.ordered, hs); break;
      default: e = miq::launch_f32_grad_direct(g, bg, x, dy, dw, hs); break;
    }
    if (e != hipSuccess) return hip_fail(e, "fp32 grad launch");
  }
  if (dbias != nullptr && static_cast<long long>(g.K) * bg.By * bg.Bx > 0) {
    float* part = reinterpret_cast<float*>(static_cast<char*>(ws) + ch.dbias_off);
    e = miq::launch_f32_block_dbias(g, bg, dy, dbias, bias_mode, part, hs);
    if (e != hipSuccess) return hip_fail(e, "fp32 bias gradient launch");
  }
  return MIQ_OK;
}

// Grow-only device workspace per device for miq_grad_nhwc_f32 and miq_block_grad_nhwc_f32
// (the reference keeps one static workspace for its fp32 path, cuda_kernels.cu:155-158, grown
// by ensure_capacity).  As the float-code workspace, it grows without freeing or waiting:
// retired buffers stay allocated until the process ends.  Calls that overlap on one device
// share it and race, as the reference's do.
constexpr int kMaxDevices = 64;
std::mutex g_grad_ws_m;
miq::GrowBuffer g_grad_ws[kMaxDevices];

int cached_workspace(size_t bytes, void** out) {
  *out = nullptr;
  if (bytes == 0) return MIQ_OK;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(MIQ_ERR_UNSUPPORTED, "device index beyond the workspace table");
  std::lock_guard<std::mutex> lock(g_grad_ws_m);
  HipAlloc alloc;
  if (miq::grow_buffer(g_grad_ws[dev], bytes, alloc, out) != 0) return hip_fail(alloc.err, "hipMalloc of the grad workspace");
  return MIQ_OK;
}

// The kernel family a pass runs (miq_plan_f32, miq_plan_block_f32), with 16-byte aligned tensors.
int plan_f32(int32_t op, const miq::Geom& g, const miq::BlockGeom& bg, int32_t algo, int32_t* kernel) {
  static const float kAligned[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const void* al = static_cast<const void*>(kAligned);
  const bool dense = bg.By == 1 && bg.Bx == 1;
  std::string why;
  switch (op) {
    case 0:  // fprop: the order of fprop_f32
      switch (algo) {
        case MIQ_ALGO_AUTO:
          *kernel = miq::f32_igemm_eligible(g, bg, al, al, nullptr) ? (g.Kg <= 32 ? MIQ_F32_IGEMM32 : MIQ_F32_IGEMM)
                    : dense && miq::f32_depthwise_eligible(g, al, al) ? MIQ_F32_DEPTHWISE
                                                                       : MIQ_F32_DIRECT;
          return MIQ_OK;
        case MIQ_ALGO_DIRECT: *kernel = MIQ_F32_DIRECT; return MIQ_OK;
        case MIQ_ALGO_IGEMM:
          if (!miq::f32_igemm_eligible(g, bg, al, al, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
          *kernel = g.Kg <= 32 ? MIQ_F32_IGEMM32 : MIQ_F32_IGEMM;
          return MIQ_OK;
        default: return fail(MIQ_ERR_INVALID_ARGUMENT, "fp32 convolution algo must be AUTO, DIRECT or IGEMM");
      }
    case 1:  // bprop: the order of bprop_f32
      switch (algo) {
        case MIQ_ALGO_AUTO:
          *kernel = miq::f32_bprop_igemm_eligible(g, bg, al, al, nullptr)            ? MIQ_F32_BPROP_IGEMM
                    : dense && miq::f32_depthwise_bprop_eligible(g, al, al) ? MIQ_F32_DEPTHWISE
                                                                             : MIQ_F32_DIRECT;
          return MIQ_OK;
        case MIQ_ALGO_DIRECT: *kernel = MIQ_F32_DIRECT; return MIQ_OK;
        case MIQ_ALGO_IGEMM:
          if (!miq::f32_bprop_igemm_eligible(g, bg, al, al, &why)) return fail(MIQ_ERR_UNSUPPORTED, why);
          *kernel = MIQ_F32_BPROP_IGEMM;
          return MIQ_OK;
        default: return fail(MIQ_ERR_INVALID_ARGUMENT, "fp32 bprop algo must be AUTO, DIRECT or IGEMM");
      }
    case 2: {  // grad: grad_choose
      GradChoice ch;
      const int st = grad_choose(g, bg, al, al, algo, false, &ch);
      if (st != MIQ_OK) return st;
      *kernel = ch.kind == kGradDepthwise ? MIQ_F32_GRAD_DEPTHWISE : ch.kind == kGradIgemm ? MIQ_F32_GRAD_IGEMM
                                                                                          : MIQ_F32_DIRECT;
      return MIQ_OK;
    }
    default: return fail(MIQ_ERR_INVALID_ARGUMENT, "op must be 0 (fprop), 1 (bprop) or 2 (grad)");
  }
}

}  // namespace

namespace miq {

int report_error(int status, const std::string& msg) { return fail(status, msg); }

int grad_f32_check(const float* x, const float* dy, float* dw, int32_t n, int32_t h, int32_t wdt, int32_t c, int32_t r,
                   int32_t s, int32_t k, const miq_conv2d_params* p, int32_t algo, size_t* ws_bytes) {
  *ws_bytes = 0;
  miq::Geom g;
  int st = infer_geom(n, h, wdt, c, r, s, k, p, &g);
  if (st != MIQ_OK) return st;
  GradChoice ch{};
  st = grad_validate(x, dy, dw, g, miq::dense_blocks(g), nullptr, 0, algo, &ch);
  *ws_bytes = st == MIQ_OK ? ch.ws_bytes : 0;
  return st;
}

}  // namespace miq

extern "C" {

int miq_grad_nhwc_f32_workspace_size(int32_t n, int32_t h, int32_t wdt, int32_t c, int32_t r, int32_t s, int32_t k,
                                     const miq_conv2d_params* p, int32_t algo, size_t* bytes) {
  if (bytes == nullptr) return fail(MIQ_ERR_NULL_POINTER, "bytes pointer is NULL");
  *bytes = 0;
  miq::Geom g;
  int st = infer_geom(n, h, wdt, c, r, s, k, p, &g);
  if (st != MIQ_OK) return st;
  // the choice of kernel for AUTO also depends on the alignment of x and dy: report the
  // larger of the aligned and unaligned choices
  GradChoice aligned{}, unaligned{};
  const float* a16 = reinterpret_cast<const float*>(static_cast<uintptr_t>(256));
  const float* a4 = reinterpret_cast<const float*>(static_cast<uintptr_t>(260));
  const miq::BlockGeom bg = miq::dense_blocks(g);
  st = grad_choose(g, bg, a16, a16, algo, false, &aligned);
  if (st != MIQ_OK) return st;
  st = grad_choose(g, bg, a4, a4, algo, false, &unaligned);
  if (st != MIQ_OK) return st;
  *bytes = aligned.ws_bytes > unaligned.ws_bytes ? aligned.ws_bytes : unaligned.ws_bytes;
  return MIQ_OK;
}

int miq_grad_nhwc_f32_ws(const float* x, const float* dy, float* dw, int32_t n, int32_t h, int32_t wdt, int32_t c,
                         int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p, int32_t algo, void* workspace,
                         size_t workspace_bytes, void* stream) {
  miq::Geom g;
  int st = infer_geom(n, h, wdt, c, r, s, k, p, &g);
  if (st != MIQ_OK) return st;
  const miq::BlockGeom bg = miq::dense_blocks(g);
  GradChoice ch{};
  st = grad_validate(x, dy, dw, g, bg, nullptr, 0, algo, &ch);
  if (st != MIQ_OK) return st;
  if (ch.ws_bytes > 0 && workspace == nullptr) return fail(MIQ_ERR_NULL_POINTER, "workspace pointer is NULL");
  if (workspace_bytes < ch.ws_bytes) {
    return fail(MIQ_ERR_INVALID_ARGUMENT, "workspace is smaller than miq_grad_nhwc_f32_workspace_size reports");
  }
  return grad_launch(g, bg, ch, x, dy, dw, nullptr, 0, workspace, stream);
}

int miq_grad_nhwc_f32(const float* x, const float* dy, float* dw, int32_t n, int32_t h, int32_t wdt, int32_t c,
                      int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p, int32_t algo, void* stream) {
  miq::Geom g;
  int st = infer_geom(n, h, wdt, c, r, s, k, p, &g);
  if (st != MIQ_OK) return st;
  const miq::BlockGeom bg = miq::dense_blocks(g);
  GradChoice ch{};
  st = grad_validate(x, dy, dw, g, bg, nullptr, 0, algo, &ch);
  if (st != MIQ_OK) return st;
  void* ws = nullptr;
  if (filt_elems(g) > 0) {
    st = cached_workspace(ch.ws_bytes, &ws);
    if (st != MIQ_OK) return st;
  }
  return grad_launch(g, bg, ch, x, dy, dw, nullptr, 0, ws, stream);
}

int miq_block_grad_nhwc_f32(const float* x, const float* dy, float* dw, int32_t n, int32_t h, int32_t wdt, int32_t c,
                            int32_t r, int32_t s, int32_t k, const miq_block_conv2d_params* p, float* dbias,
                            int32_t bias_mode, int32_t algo, void* stream) {
  miq::Geom g;
  miq::BlockGeom bg;
  int st = infer_block_geom(n, h, wdt, c, r, s, k, p, &g, &bg);
  if (st != MIQ_OK) return st;
  GradChoice ch{};
  st = grad_validate(x, dy, dw, g, bg, dbias, bias_mode, algo, &ch);
  if (st != MIQ_OK) return st;
  void* ws = nullptr;
  st = cached_workspace(ch.ws_bytes, &ws);
  if (st != MIQ_OK) return st;
  return grad_launch(g, bg, ch, x, dy, dw, dbias, bias_mode, ws, stream);
}

int miq_plan_f32(int32_t op, int32_t n, int32_t h, int32_t wdt, int32_t c, int32_t r, int32_t s, int32_t k,
                 const miq_conv2d_params* p, int32_t algo, int32_t* kernel) {
  if (kernel == nullptr) return fail(MIQ_ERR_NULL_POINTER, "kernel pointer is NULL");
  miq::Geom g;
  const int st = infer_geom(n, h, wdt, c, r, s, k, p, &g);
  if (st != MIQ_OK) return st;
  return plan_f32(op, g, miq::dense_blocks(g), algo, kernel);
}

int miq_plan_block_f32(int32_t op, int32_t n, int32_t h, int32_t wdt, int32_t c, int32_t r, int32_t s, int32_t k,
                       const miq_block_conv2d_params* p, int32_t algo, int32_t* kernel) {
  if (kernel == nullptr) return fail(MIQ_ERR_NULL_POINTER, "kernel pointer is NULL");
  miq::Geom g;
  miq::BlockGeom bg;
  const int st = infer_block_geom(n, h, wdt, c, r, s, k, p, &g, &bg);
  if (st != MIQ_OK) return st;
  return plan_f32(op, g, bg, algo, kernel);
}

int miq_bmm_i32(const int32_t* A, const int32_t* B, int32_t* C, int32_t batch, int32_t M, int32_t N, int32_t K,
                int32_t trans_a, int32_t trans_b, void* stream) {
  if (batch < 0 || M < 0 || N < 0 || K < 0) return fail(MIQ_ERR_INVALID_ARGUMENT, "bmm extents must be >= 0");
  constexpr int32_t kMaxExtent = 0x7fffffff - 64;  // tile and chunk indices stay in int32
  if (M > kMaxExtent || N > kMaxExtent || K > kMaxExtent) {
    return fail(MIQ_ERR_UNSUPPORTED, "bmm extents must be <= 2^31 - 65");
  }
  if (batch == 0 || M == 0 || N == 0) return MIQ_OK;
  if (C == nullptr) return fail(MIQ_ERR_NULL_POINTER, "bmm output pointer C is NULL");
  if (K > 0 && A == nullptr) return fail(MIQ_ERR_NULL_POINTER, "bmm input pointer A is NULL");
  if (K > 0 && B == nullptr) return fail(MIQ_ERR_NULL_POINTER, "bmm input pointer B is NULL");
  const long long tiles = ((M + 127LL) / 128) * ((N + 63LL) / 64);
  if (tiles > (1LL << 22)) return fail(MIQ_ERR_UNSUPPORTED, "bmm matrix has more than 2^22 128x64 output tiles");
  const hipError_t e = miq::launch_i32_gemm(A, B, C, batch, M, N, K, trans_a != 0, trans_b != 0,
                                            static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "int32 bmm launch");
  return MIQ_OK;
}

void bmm_matmul_i32(const int32_t* A, const int32_t* B, int32_t* C, int batch, int M, int N, int K, int trans_a,
                    int trans_b) {
  (void)miq_bmm_i32(A, B, C, batch, M, N, K, trans_a, trans_b, nullptr);
}

}  // extern "C"
