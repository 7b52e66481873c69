// Internal interface between the C-ABI front end (qconv_capi.cpp) and the HIP kernel
// translation units.  Not installed; callers use include/miq_qconv.h.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

struct miq_conv2d_params;  // include/miq_qconv.h

namespace miq {

// Validated geometry of one grouped 2-D convolution, NHWC input / KRSC filter.
struct Geom {
  int N, H, W, C;      // input
  int K, R, S;         // filter (K output channels, R x S taps)
  int Ho, Wo;          // output spatial size
  int ph, pw;          // padding
  int sh, sw;          // stride
  int dh, dw;          // dilation
  int G, Cg, Kg;       // groups, input / output channels per group
};

// Output stage of the int8 kernels.
enum Epi : int {
  kEpiI8 = 0,     // requantized int8
  kEpiAcc32 = 1,  // raw int32 accumulators
  kEpiF32 = 2,    // dequantized fp32 view
  kEpiQi32 = 3,   // int32 of the float-code route: offset codes' corrections added (stream kernel only)
};

// Requantization inputs; act_scale = in_scale / out_scale, computed on the host.
struct Requant {
  const int32_t* bias;    // int32[K] or nullptr
  const float* wscale;    // float[K] (unused for kEpiAcc32)
  float act_scale;
  int relu;
};

// Blocked-filter geometry; By == Bx == 1 describes a plain KRSC filter.
struct BlockGeom {
  int By, Bx;          // filter blocks
  int bho, bwo;        // output rows / cols per block
};

enum QpKind : int { kQpU8 = 0, kQpS5 = 1 };

// Division by a launch-constant divisor d >= 1 for numerators 0 <= n < 2^31, as one
// multiply-high, one add and one shift (Granlund & Montgomery, "Division by invariant
// integers using multiplication", 1994): s = ceil(log2 d), m = floor(2^32 (2^s - d) / d) + 1,
// n / d = (mulhi(n, m) + n) >> s.
struct FastDiv {
  uint32_t d, m, s;
};

inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t s = 0;
  while ((uint64_t{1} << s) < d) ++s;
  const uint64_t m = ((uint64_t{1} << 32) * ((uint64_t{1} << s) - d)) / d + 1;
  return FastDiv{d, static_cast<uint32_t>(m), s};
}

inline uint32_t fastdiv_host(uint32_t n, const FastDiv& f) {
  const uint32_t t = static_cast<uint32_t>((static_cast<uint64_t>(n) * f.m) >> 32);
  return (t + n) >> f.s;
}

// int32 accumulators on float codes with per-sample input zero points (compat surface).
hipError_t launch_qi32_direct(const Geom& g, const BlockGeom& bg, QpKind qp, const float* x, const float* w,
                              int32_t* y, const void* in_qp, const void* f_qp, hipStream_t stream);

// int32 accumulators on float codes on the int8 matrix cores (digits of the centred codes):
// plain or blocked filters, any C/groups, 4-byte aligned x and w, a non-empty image.
bool qi32_igemm_eligible(const Geom& g, const BlockGeom& bg, const void* x, const void* w, std::string* why);
hipError_t launch_qi32_igemm(const Geom& g, const BlockGeom& bg, QpKind qp, const float* x, const float* w, int32_t* y,
                             const void* in_qp, const void* f_qp, hipStream_t stream);

// int32 accumulators on float codes on the int8 row-band structure (codes staged once per band
// as offset int8 values, filter in registers): plain filters, (C/groups) % 64 == 0,
// (K/groups) % 16 == 0, stride_w == 1, Wo <= 64, R*S*C/groups <= 576, 16-byte aligned x, w, y.
// Exact for any codes: a workgroup whose codes leave the parameter type's int8 window computes
// directly.
bool qi32_band_eligible(const Geom& g, const BlockGeom& bg, const void* x, const void* w, const void* y,
                        std::string* why);
// Device bytes of the workspace launch_qi32_band takes (the filter converted once per call to
// int8 MFMA fragments, and range flags); the caller keeps it unused by other work until the
// launches on `stream` have completed.
size_t qi32_band_workspace_bytes(const Geom& g, const BlockGeom& bg);
hipError_t launch_qi32_band(const Geom& g, const BlockGeom& bg, QpKind qp, const float* x, const float* w, int32_t* y,
                            const void* in_qp, const void* f_qp, void* ws, hipStream_t stream);

// int32 accumulators on float codes through the int8 stream kernel (prepass to a padded
// offset-int8 image and int8 filter in the workspace, the stream kernel with the offset
// corrections, an exact direct pass only when a code leaves int8): plain filters on the shapes
// the stream kernel takes after padding is folded into the image.
bool qi32_route_eligible(const Geom& g, const BlockGeom& bg, const void* x, const void* w, const void* y,
                         std::string* why);
size_t qi32_route_workspace_bytes(const Geom& g);
hipError_t launch_qi32_route(const Geom& g, QpKind qp, const float* x, const float* w, int32_t* y, const void* in_qp,
                             const void* f_qp, void* ws, hipStream_t stream);

// int32 accumulators on float codes through the space-to-depth stem kernel (stride-2
// thin-channel layers): a prepass to a padded offset-int8 image (rows padded to a multiple of
// 16 bytes) and int8 filter in the workspace, the s2d kernel with the offset corrections, an
// exact direct pass only when a code leaves int8.
bool qi32_stem_route_eligible(const Geom& g, const BlockGeom& bg, const void* x, const void* w, const void* y,
                              std::string* why);
size_t qi32_stem_route_workspace_bytes(const Geom& g);
hipError_t launch_qi32_stem_route(const Geom& g, QpKind qp, const float* x, const float* w, int32_t* y,
                                  const void* in_qp, const void* f_qp, void* ws, hipStream_t stream);

// int8 VALU direct convolution: any geometry.
hipError_t launch_i8_direct(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                            hipStream_t stream);

// int8 MFMA implicit GEMM: (C/groups) % 16 == 0, stride/dilation >= 1, padding >= 0.
bool igemm_eligible(const Geom& g, const void* x, const void* w, const void* y, Epi epi, std::string* why);
hipError_t launch_i8_igemm(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                           hipStream_t stream);

// int8 MFMA row-band kernel, filter in registers: (C/groups) % 64 == 0, (K/groups) % 16 == 0,
// stride_w == 1, Wo <= 64, R*S*C/groups <= 576.
bool band_eligible(const Geom& g, const void* x, const void* w, const void* y, const Requant& rq, Epi epi,
                   std::string* why);
hipError_t launch_i8_band(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                          hipStream_t stream);

// The stream kernel on offset int8 codes (x' = code - o, w' = code - o) of a padded input (g has
// no padding), int32 out:  y = sum x'w' + dx[n] * T[k] + Kdim * dx[n] * dw + dw * W(p), with
// T[k] the sum of filter row k, W(p) the sum of the pixel's window, and qrec[4n .. 4n + 3] =
// {dx[n], dw, Kdim * dx[n] * dw, 0} (mod 2^32).
hipError_t launch_i8_stream_qi32(const Geom& g, const int8_t* x, const int8_t* w, const int32_t* T,
                                 const int32_t* qrec, int32_t* y, hipStream_t stream);

// int8 MFMA row-band kernel over virtual pixels (stride 1), filter in registers:
// (C/groups) % 64 == 0, (K/groups) % 64 == 0, R*S*C/groups <= 576.
bool flat_eligible(const Geom& g, const void* x, const void* w, const void* y, const Requant& rq, Epi epi,
                   std::string* why);
hipError_t launch_i8_flat(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                          hipStream_t stream);

// int8 MFMA row-band kernel whose input rows stream into LDS under the matrix instructions
// (loader wave, per-row LDS flags): int8 output, groups 1, C == K == 64, stride 1, 3x3 or 1x1,
// Wo % 8 == 0.
bool pipe_eligible(const Geom& g, const void* x, const void* w, const void* y, const Requant& rq, Epi epi,
                   std::string* why);
hipError_t launch_i8_pipe(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                          hipStream_t stream);

// int8 MFMA stem kernel over a space-to-depth copy of the input (stride 2, 1 <= C <= 4, groups 1,
// K % 64 == 0, ceil(R/2) * ceil(S/2) <= 16, int8 output).
bool stem_s2d_eligible(const Geom& g, const void* x, const void* w, const void* y, const Requant& rq, Epi epi,
                       std::string* why);
hipError_t launch_i8_stem_s2d(const Geom& g, const int8_t* x, const int8_t* w, int8_t* y, const Requant& rq,
                              hipStream_t stream);
// The same kernel on offset codes with int32 outputs (the float-code stem route): `g` is the
// padded problem (padding 0, its own Ho and Wo), T the filter row sums, qrec the per-image
// records {dx, dw, Kdim * dx * dw, 0}.
bool stem_s2d_qi32_plan_ok(const Geom& g, std::string* why);
hipError_t launch_stem_s2d_qi32(const Geom& g, const int8_t* x, const int8_t* w, const int32_t* T,
                                const int32_t* qrec, int32_t* y, hipStream_t stream);

// int8 MFMA pointwise kernel (1x1, stride 1, no padding, groups 1, C 64 or 128, K % 64 == 0):
// a GEMM over the flattened pixels with the input streamed into LDS by a loader wave.
bool pointwise_eligible(const Geom& g, const void* x, const void* w, const void* y, const Requant& rq, Epi epi,
                        std::string* why);
hipError_t launch_i8_pointwise(const Geom& g, const int8_t* x, const int8_t* w, int8_t* y, const Requant& rq,
                               hipStream_t stream);

// int8 MFMA kernel with the filter streamed through LDS: (C/groups) % 64 == 0,
// (K/groups) % 128 == 0, stride_w <= 4.
bool stream_eligible(const Geom& g, const void* x, const void* w, const void* y, const Requant& rq, Epi epi,
                     std::string* why);
hipError_t launch_i8_stream(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                            hipStream_t stream);

// int8 convolution on the vector ALU (v_dot4_i32_i8), any group shape: the filter tile
// (r * s * ceil(Cg/4) * up to 32 channels dwords) must fit in 64 KB of LDS.
bool dot4_eligible(const Geom& g, std::string* why);
// AUTO's choice of it: few output channels per group (<= 8) on a 1x1 or small filter, where it
// measured faster than the implicit GEMM
bool dot4_preferred(const Geom& g);
hipError_t launch_i8_dot4(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                          hipStream_t stream);

// int8 MFMA thin-channel kernel for stems: groups == 1, C < 16.
bool stem_eligible(const Geom& g, const void* x, const void* w, const void* y, Epi epi, std::string* why);
hipError_t launch_i8_stem(const Geom& g, Epi epi, const int8_t* x, const int8_t* w, void* y, const Requant& rq,
                          hipStream_t stream);

// fp32 NHWC convolution: MFMA implicit GEMM for (C/groups) % 4 == 0 with 16-byte aligned x
// and w and a non-empty image; the direct kernel (reference CPU loop order) for any shape.
// bg: the filter's block grid (dense_blocks(g) for a plain KRSC filter); bias (K * By * Bx
// floats, bias_mode 0 per block or 1 shared) may be nullptr.
inline BlockGeom dense_blocks(const Geom& g) { return BlockGeom{1, 1, g.Ho, g.Wo}; }
bool f32_igemm_eligible(const Geom& g, const BlockGeom& bg, const void* x, const void* w, std::string* why);
hipError_t launch_f32_igemm(const Geom& g, const BlockGeom& bg, const float* x, const float* w, const float* bias,
                            int bias_mode, float* y, hipStream_t stream);
hipError_t launch_f32_direct(const Geom& g, const BlockGeom& bg, const float* x, const float* w, const float* bias,
                             int bias_mode, float* y, hipStream_t stream);
// fp32 depthwise (C/groups == K/groups == 1, C % 4 == 0, R*S*C <= 8192, 16-byte aligned x and y),
// four channels per thread in the reference loop's order: bit-exact like the direct kernel.
bool f32_depthwise_eligible(const Geom& g, const void* x, const void* y);
hipError_t launch_f32_depthwise(const Geom& g, const float* x, const float* w, float* y, hipStream_t stream);
// fp32 dx and dw in the reference CPU loop orders (one thread per output element).
bool f32_depthwise_bprop_eligible(const Geom& g, const void* dy, const void* dx);
hipError_t launch_f32_depthwise_bprop(const Geom& g, const float* dy, const float* w, float* dx, hipStream_t stream);
hipError_t launch_f32_bprop_direct(const Geom& g, const BlockGeom& bg, const float* dy, const float* w, float* dx,
                                   hipStream_t stream);
// fp32 dx of a stride-1 convolution on the MFMA implicit GEMM (the forward kernel over dy with
// the flipped, channel-transposed filter): (K/groups) % 4 == 0, 16-byte aligned dy.
bool f32_bprop_igemm_eligible(const Geom& g, const BlockGeom& bg, const void* dy, const void* w, std::string* why);
hipError_t launch_f32_bprop_igemm(const Geom& g, const BlockGeom& bg, const float* dy, const float* w, float* dx,
                                  hipStream_t stream);
hipError_t launch_f32_grad_direct(const Geom& g, const BlockGeom& bg, const float* x, const float* dy, float* dw,
                                  hipStream_t stream);
// fp32 dw on the MFMA (pixel range split over workgroups): any non-empty shape.  ordered: the
// splits' partial tiles go to `ws` (f32_grad_igemm_workspace bytes, none for one split) and
// are summed in split order, the same result on every call; otherwise they are added into dw
// with float atomics after a zero fill (ws unused), whose order varies from run to run.
bool f32_grad_igemm_eligible(const Geom& g, const BlockGeom& bg, std::string* why);
size_t f32_grad_igemm_workspace(const Geom& g, const BlockGeom& bg);
hipError_t launch_f32_grad_igemm(const Geom& g, const BlockGeom& bg, const float* x, const float* dy, float* dw,
                                 float* ws, bool ordered, hipStream_t stream);
// Bias gradient of the blocked convolution: dbias (K * By * Bx floats, bias_mode 0 per block or
// 1 shared) = the sum of dy over every output position of each block, in a fixed order, through
// f32_block_dbias_workspace bytes of `ws` (nonzero for any non-empty dy).
size_t f32_block_dbias_workspace(const Geom& g, const BlockGeom& bg);
hipError_t launch_f32_block_dbias(const Geom& g, const BlockGeom& bg, const float* dy, float* dbias, int bias_mode,
                                  float* ws, hipStream_t stream);
// fp32 depthwise dw (C/groups == K/groups == 1, C % 4 == 0, R*S <= 16, 16-byte aligned x and dy):
// pixel runs per thread; ordered: partial sums of every run to `ws`
// (f32_depthwise_grad_workspace bytes) summed in run order; otherwise float atomics into dw.
bool f32_depthwise_grad_eligible(const Geom& g, const void* x, const void* dy);
// Validation of an fp32 grad call exactly as miq_grad_nhwc_f32_ws does it (status and message
// left like an entry point's), and the workspace bytes it needs for these pointers.
int grad_f32_check(const float* x, const float* dy, float* dw, int32_t n, int32_t h, int32_t wdt, int32_t c, int32_t r,
                   int32_t s, int32_t k, const ::miq_conv2d_params* p, int32_t algo, size_t* ws_bytes);
// Records `msg` as the calling thread's miq_last_error_message() and returns `status`.
int report_error(int status, const std::string& msg);
size_t f32_depthwise_grad_workspace(const Geom& g);
hipError_t launch_f32_depthwise_grad(const Geom& g, const float* x, const float* dy, float* dw, float* ws,
                                     bool ordered, hipStream_t stream);

// int32 batched GEMM (wrap-around arithmetic) on the int8 matrix cores; extents already
// validated (>= 0), pointers non-null where the extents need them.
hipError_t launch_i32_gemm(const int32_t* A, const int32_t* B, int32_t* C, int batch, int M, int N, int K, bool ta,
                           bool tb, hipStream_t stream);

#if defined(__HIPCC__)
__device__ __forceinline__ int fdiv(int n, const FastDiv& f) {
  const uint32_t un = static_cast<uint32_t>(n);
  return static_cast<int>((__umulhi(un, f.m) + un) >> f.s);
}

// ---- epilogue arithmetic shared by every int8 kernel --------------------------------
// Each step is one IEEE-754 single operation with round-to-nearest-even, in this order,
// so the GPU result equals the host restatement bit for bit (no contraction: the
// translation units are compiled with -ffp-contract=off and no step is a*b+c).

__device__ __forceinline__ float requant_multiplier(float act_scale, float wscale) {
  return act_scale * wscale;
}

__device__ __forceinline__ int requant_i8(int32_t acc, int32_t bias, float m, float lo) {
  const int32_t t = static_cast<int32_t>(static_cast<uint32_t>(acc) + static_cast<uint32_t>(bias));
  const float v = static_cast<float>(t) * m;
  float q = __builtin_rintf(v);
  q = (q >= lo) ? q : lo;          // NaN -> lo
  q = (q > 127.0f) ? 127.0f : q;
  return static_cast<int>(q);
}

__device__ __forceinline__ float dequant_f32(int32_t acc, int32_t bias, float m, int relu) {
  const int32_t t = static_cast<int32_t>(static_cast<uint32_t>(acc) + static_cast<uint32_t>(bias));
  float v = static_cast<float>(t) * m;
  if (relu) v = (v > 0.0f) ? v : 0.0f;  // NaN and -0 -> +0
  return v;
}
#endif

}  // namespace miq
