/*
 * miq_qconv.h - C-ABI of the MI355X (gfx950) quantized NHWC convolution library.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream, returns a
 * miq_status code and never throws.  The C++ drop-in surface (conv_types.h) and the
 * Python binding (my_own_cnn_amd) are thin layers over these functions.
 *
 * Conventions
 *   - Tensors are dense and live in device memory owned by the caller:
 *       input  x: NHWC, n*h*w*c elements
 *       filter w: KRSC, k*r*s*(c/groups) elements
 *       output y: NHWC, n*ho*wo*k elements, fully overwritten
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream).  Calls are
 *     asynchronous with respect to the host; the caller synchronises.
 *   - Arguments are validated on the host before anything is enqueued; a failed
 *     validation returns a non-zero status and leaves the output untouched.
 *   - Device memory the library allocates itself: the entry points with the reference's
 *     signatures that need a workspace and have no argument for one keep grow-only buffers
 *     (the float-code row-band and stream paths one per (device, stream), at most 64 such
 *     pairs; the fp32 filter gradient one per device), allocated with hipMalloc on first use
 *     and when a larger problem arrives.  A grown-out buffer is kept, not freed, until the
 *     process ends, and no call synchronises.  Each has a form that takes the caller's
 *     workspace and allocates nothing (miq_fprop_nhwc_qi32_ws, miq_grad_nhwc_f32_ws).  The
 *     32 MiB array of miq_grad_nhwc_f32_noalloc is part of the library's device code and is
 *     allocated when that code is loaded on a device.  Nothing else is allocated, and no
 *     other global state changes, so calls on different streams may overlap.
 *   - miq_last_error_message() returns the text of the last non-OK status raised on
 *     the calling thread.
 */
#ifndef MIQ_QCONV_H_
#define MIQ_QCONV_H_

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MIQ_VERSION 100 /* 1.0.0 */

typedef enum miq_status {
  MIQ_OK = 0,
  MIQ_ERR_NULL_POINTER = 1,     /* a required pointer argument is NULL */
  MIQ_ERR_INVALID_ARGUMENT = 2, /* shape or parameter rejected (same rules as the reference) */
  MIQ_ERR_UNSUPPORTED = 3,      /* valid problem the requested algorithm cannot run */
  MIQ_ERR_HIP = 4               /* a HIP runtime call or kernel launch failed */
} miq_status;

/* Kernel families of the int8 entry points (miq_qconv_desc.algo). */
typedef enum miq_algo {
  MIQ_ALGO_AUTO = 0,   /* pick by shape: pointwise kernel (int8 output), else band kernel, else flat
                          kernel, else stream kernel, else the dot4
                          kernel for <= 8 output channels per group on 1x1 or small filters, else
                          implicit GEMM, else the space-to-depth stem kernel (int8 output), else
                          stem kernel for thin C, else direct */
  MIQ_ALGO_DIRECT = 1, /* VALU direct convolution: any shape, bandwidth-bound fallback */
  MIQ_ALGO_IGEMM = 2,  /* int8 MFMA implicit GEMM: needs (c/groups) % 16 == 0, 16-byte aligned tensors */
  MIQ_ALGO_STEM = 3,   /* int8 MFMA thin-channel kernel: c/groups < 16, groups == 1 */
  MIQ_ALGO_BAND = 4    /* int8 MFMA row-band kernel with the filter held in registers: needs
                          (c/groups) % 64 == 0, (k/groups) % 16 == 0, stride_w == 1, output width
                          <= 64, r*s*c/groups <= 576, 16-byte aligned tensors, bias and scales */,
  MIQ_ALGO_STREAM = 5, /* int8 MFMA row-band kernel with the filter streamed through LDS: needs
                          (c/groups) % 64 == 0, (k/groups) % 128 == 0, stride_w <= 4, input rows of a
                          band that fit in LDS, 16-byte aligned tensors, bias and scales */
  MIQ_ALGO_ATOMIC = 6, /* fp32 grad only: AUTO's kernels with the split partial sums added by float
                          atomics (no workspace; the summation order varies from run to run) */
  MIQ_ALGO_FLAT = 7    /* int8 MFMA row-band kernel over virtual pixels (rows padded to the input
                          halo's width), filter held in registers: needs stride 1, (c/groups) % 64
                          == 0, (k/groups) % 64 == 0, r*s*c/groups <= 576, a band's input rows that
                          fit in LDS, 16-byte aligned tensors, bias and scales */,
  MIQ_ALGO_DOT4 = 8    /* int8 vector-ALU kernel (v_dot4_i32_i8, no matrix instructions): any shape
                          whose filter tile, r*s*ceil(c/groups/4) x up to 32 channels dwords, fits in
                          64 KB; the bandwidth-bound fallback for thin C and few output channels */,
  MIQ_ALGO_PIPE = 9    /* int8 MFMA row-band kernel whose input rows stream into LDS under the matrix
                          instructions (a loader wave publishes each row): int8 output only, groups
                          1, c == k == 64, stride 1, a 3x3 or 1x1 filter, output width % 8 == 0,
                          16-byte aligned tensors, bias and scales */,
  MIQ_ALGO_POINTWISE = 10 /* int8 MFMA GEMM over the flattened pixels of a 1x1 convolution, input
                          streamed into LDS by a loader wave: int8 output only, groups 1, stride 1,
                          no padding, c 64 or 128, k % 64 == 0, 16-byte aligned tensors, bias and
                          scales */,
  MIQ_ALGO_STEM_S2D = 11 /* int8 MFMA stem kernel over a space-to-depth copy of the input built in LDS:
                          int8 output only, groups 1, stride 2, dilation 1, 1 <= c <= 4, k % 64 ==
                          0, ceil(r/2) * ceil(s/2) <= 16, w*c % 16 == 0, output width <= 112,
                          16-byte aligned tensors, bias and scales */
} miq_algo;

/* Same member order and layout as Conv2DParams (/root/reference/src/conv_types.h:21-29). */
typedef struct miq_conv2d_params {
  int32_t pad_h;
  int32_t pad_w;
  int32_t stride_h;
  int32_t stride_w;
  int32_t dilation_h;
  int32_t dilation_w;
  int32_t groups;
} miq_conv2d_params;

/* Same layout as BlockConv2DParams (/root/reference/src/conv_types.h:31-35). */
typedef struct miq_block_conv2d_params {
  miq_conv2d_params conv;
  int32_t block_by;
  int32_t block_bx;
} miq_block_conv2d_params;

/* Byte layout of QuantizationParameters<LinQuantU8> (nnalgebra_quantization.h:29-34):
 * 12 bytes, zero_point at 0, scale at 4, symmetric at 8. */
typedef struct miq_qparams_u8 {
  uint8_t zero_point;
  float scale;
  uint8_t symmetric;
} miq_qparams_u8;

/* Byte layout of QuantizationParameters<LinQuantS5> (nnalgebra_quantization.h:36-41):
 * 8 bytes, zero_point at 0, n_bins at 1, scale at 4. */
typedef struct miq_qparams_s5 {
  int8_t zero_point;
  uint8_t n_bins;
  float scale;
} miq_qparams_s5;

/* Problem description of the native int8 convolution.
 *   y[n,ho,wo,k] = requant( sum_{r,s,ci} x[n, ho*sh-ph+r*dh, wo*sw-pw+s*dw, g*c/groups+ci]
 *                                        * w[k, r, s, ci] )
 * over in-bounds taps only (padded taps contribute 0), g = k / (k_total/groups).
 * Requantization of one int32 accumulator `acc` of output channel k:
 *   a  = in_scale / out_scale                (fp32, computed once on the host)
 *   m  = a * w_scale[k]                      (fp32 multiply, round to nearest even)
 *   v  = (float)(acc + bias[k]) * m          (int32 wrap-around add, exact-RNE convert, fp32 multiply)
 *   q  = rint(v) (ties to even), then q < lo -> lo (NaN -> lo), q > 127 -> 127
 *   lo = 0 when relu != 0, else -128.
 * Zero points are 0 (symmetric int8, nnalgebra::DataType::LinQuantI8). */
typedef struct miq_qconv_desc {
  int32_t n, h, w, c;      /* input NHWC */
  int32_t k, r, s;         /* filter: k output channels, r x s taps, c/groups input channels */
  miq_conv2d_params conv;  /* padding, stride, dilation, groups */
  int32_t relu;            /* non-zero: clamp the output below at 0 */
  float in_scale;          /* real value of one input code step */
  float out_scale;         /* real value of one output code step */
  int32_t algo;            /* miq_algo; MIQ_ALGO_AUTO selects by shape */
} miq_qconv_desc;

/* ---- library information (host only) ---------------------------------------------- */

int miq_version(void);
const char* miq_status_string(int status);
const char* miq_last_error_message(void);

/* ---- shape inference (host only, no GPU access) ------------------------------------ */

/* Output spatial size with the validation rules of infer_conv_shape
 * (/root/reference/src/conv_types.h:125-146). */
int miq_conv2d_output_shape(int32_t n, int32_t h, int32_t w, int32_t c,
                            int32_t r, int32_t s, int32_t k,
                            const miq_conv2d_params* p, int32_t* ho, int32_t* wo);

/* Output size and per-block extent with the rules of infer_block_conv_shape
 * (/root/reference/src/conv_types.h:148-169). */
int miq_block_conv2d_output_shape(int32_t n, int32_t h, int32_t w, int32_t c,
                                  int32_t r, int32_t s, int32_t k,
                                  const miq_block_conv2d_params* p, int32_t* ho, int32_t* wo,
                                  int32_t* block_ho, int32_t* block_wo);

/* Validates `d` and reports the kernel family the int8 entry points will run
 * (resolving MIQ_ALGO_AUTO).  No GPU access. */
int miq_qconv2d_plan(const miq_qconv_desc* d, int32_t* algo);

/* ---- int32-accumulator convolution on quantized float codes ------------------------ */
/* acc = sum over in-bounds taps of (int32(x) - zp_x[n]) * (int32(w) - zp_w), where int32()
 * truncates toward zero; in_qp is a device array of n parameter structs (one per batch
 * sample) and f_qp a device pointer to one struct. */

/* Replaces conv_quant_detail::launch_fprop_nhwc_qi32_u8 (/root/reference/src/cuda_kernels.cu:1467-1473). */
int miq_fprop_nhwc_qi32_u8(const float* x, const float* w, int32_t* y,
                           int32_t n, int32_t h, int32_t wdt, int32_t c,
                           int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p,
                           const miq_qparams_u8* in_qp, const miq_qparams_u8* f_qp, void* stream);

/* Replaces conv_quant_detail::launch_fprop_nhwc_qi32_s5 (/root/reference/src/cuda_kernels.cu:1475-1481). */
int miq_fprop_nhwc_qi32_s5(const float* x, const float* w, int32_t* y,
                           int32_t n, int32_t h, int32_t wdt, int32_t c,
                           int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p,
                           const miq_qparams_s5* in_qp, const miq_qparams_s5* f_qp, void* stream);

/* Blocked filters [K, By, Bx, R, S, C/groups]: output pixel (ho, wo) uses filter block
 * (ho / block_ho, wo / block_wo).
 * Replaces conv_quant_detail::launch_block_fprop_nhwc_qi32_u8 (/root/reference/src/cuda_kernels.cu:1483-1489). */
int miq_block_fprop_nhwc_qi32_u8(const float* x, const float* w, int32_t* y,
                                 int32_t n, int32_t h, int32_t wdt, int32_t c,
                                 int32_t r, int32_t s, int32_t k, const miq_block_conv2d_params* p,
                                 const miq_qparams_u8* in_qp, const miq_qparams_u8* f_qp, void* stream);

/* Replaces conv_quant_detail::launch_block_fprop_nhwc_qi32_s5 (/root/reference/src/cuda_kernels.cu:1491-1497). */
int miq_block_fprop_nhwc_qi32_s5(const float* x, const float* w, int32_t* y,
                                 int32_t n, int32_t h, int32_t wdt, int32_t c,
                                 int32_t r, int32_t s, int32_t k, const miq_block_conv2d_params* p,
                                 const miq_qparams_s5* in_qp, const miq_qparams_s5* f_qp, void* stream);

/* The plain-filter float-code convolution with an explicit kernel choice: qp_kind 0 takes
 * miq_qparams_u8 structs (launch_fprop_nhwc_qi32_u8's), 1 miq_qparams_s5 structs; algo is
 * MIQ_ALGO_AUTO (what the entry points above run), MIQ_ALGO_BAND (row bands, 16-byte aligned
 * x, w and y, (c/groups) % 64 == 0, (k/groups) % 16 == 0, stride_w 1, output width <= 64,
 * r*s*c/groups <= 576), MIQ_ALGO_STREAM (the int8 stream kernel on a padded offset-int8 copy
 * of the input: c/groups % 64 == 0, k/groups % 128 == 0, stride_w <= 4, 16-byte aligned
 * tensors), MIQ_ALGO_STEM_S2D (the space-to-depth stem kernel on a padded offset-int8 copy:
 * groups 1, 1 <= c <= 4, stride 2, dilation 1, k % 64 == 0, ceil(r/2) * ceil(s/2) <= 16,
 * 16-byte aligned tensors), MIQ_ALGO_IGEMM or MIQ_ALGO_DIRECT.  Results are identical for every
 * choice.  No reference counterpart: it exists for tests and benchmarks. */
int miq_fprop_nhwc_qi32_algo(int32_t qp_kind, const float* x, const float* w, int32_t* y,
                             int32_t n, int32_t h, int32_t wdt, int32_t c,
                             int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p,
                             const void* in_qp, const void* f_qp, int32_t algo, void* stream);

/* Bytes of device workspace miq_fprop_nhwc_qi32_ws needs for this shape and algo (the row-band,
 * stream and stem routes' prepass output; 0 for the others and for an empty output), for 256-byte
 * aligned tensors (misaligned ones can only take kernels that need none).  No GPU access.  No
 * reference counterpart: it sizes the caller-provided form of the workspace that
 * launch_fprop_nhwc_qi32_impl (/root/reference/src/cuda_kernels.cu:1351-1354) allocates. */
int miq_fprop_nhwc_qi32_workspace_size(int32_t n, int32_t h, int32_t wdt, int32_t c, int32_t r, int32_t s,
                                       int32_t k, const miq_conv2d_params* p, int32_t algo, size_t* bytes);

/* miq_fprop_nhwc_qi32_algo with a caller-provided device workspace of at least
 * miq_fprop_nhwc_qi32_workspace_size bytes (NULL allowed when that size is 0); allocates
 * nothing and never synchronises, so it can be recorded into a HIP graph.  Same result bits as
 * the entry points above.  The workspace must not be used by another call until this one's
 * work on `stream` has finished.  Replaces launch_fprop_nhwc_qi32_u8 / _s5
 * (/root/reference/src/cuda_kernels.cu:1467-1481) with the per-call workspace of
 * launch_fprop_nhwc_qi32_impl (:1351-1354) passed in instead. */
int miq_fprop_nhwc_qi32_ws(int32_t qp_kind, const float* x, const float* w, int32_t* y,
                           int32_t n, int32_t h, int32_t wdt, int32_t c,
                           int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p,
                           const void* in_qp, const void* f_qp, int32_t algo, void* workspace,
                           size_t workspace_bytes, void* stream);

/* The kernel the float-code entry points run for a plain-filter problem with 256-byte aligned
 * tensors: writes MIQ_ALGO_BAND, MIQ_ALGO_STREAM, MIQ_ALGO_STEM_S2D, MIQ_ALGO_IGEMM or MIQ_ALGO_DIRECT
 * to *algo.  No reference counterpart. */
int miq_plan_qi32(int32_t n, int32_t h, int32_t wdt, int32_t c, int32_t r, int32_t s, int32_t k,
                  const miq_conv2d_params* p, int32_t* algo);

/* miq_plan_qi32 for blocked filters (the kernel launch_block_fprop_nhwc_qi32 runs with
 * 256-byte aligned tensors): MIQ_ALGO_BAND (row bands inside one filter block, on the band
 * kernel's conditions for the block's width), MIQ_ALGO_IGEMM or MIQ_ALGO_DIRECT.  No reference
 * counterpart. */
int miq_plan_block_qi32(int32_t n, int32_t h, int32_t wdt, int32_t c, int32_t r, int32_t s, int32_t k,
                        const miq_block_conv2d_params* p, int32_t* algo);

/* ---- native int8 convolution ------------------------------------------------------- */
/* No reference counterpart: the int8 activation / int8 weight / int32 bias /
 * per-channel scale / int8 output surface that the reference's quantization types
 * describe but never implement.  Its int32 accumulators equal those of
 * cpu_fprop_nhwc_qi32 (/root/reference/src/cpu_ref.cpp:36-72) with zero points 0. */

/* Fused conv + bias + per-channel requantize + optional ReLU + int8 saturate.
 * bias: device int32[k] or NULL (treated as 0); w_scale: device float[k]. */
int miq_qconv2d_nhwc_i8(const miq_qconv_desc* d, const int8_t* x, const int8_t* w,
                        const int32_t* bias, const float* w_scale, int8_t* y, void* stream);

/* Raw int32 accumulators (no bias, no requantization). */
int miq_qconv2d_nhwc_i8_acc32(const miq_qconv_desc* d, const int8_t* x, const int8_t* w,
                              int32_t* acc, void* stream);

/* Dequantized fp32 view: v = (float)(acc + bias[k]) * m as defined above (no rint, no
 * clamp); with relu, v <= 0 or NaN becomes +0. */
int miq_qconv2d_nhwc_i8_dequant(const miq_qconv_desc* d, const int8_t* x, const int8_t* w,
                                const int32_t* bias, const float* w_scale, float* y, void* stream);

/* ---- fp32 convolution --------------------------------------------------------------- */

/* y = conv(x, w) in fp32, NHWC input and output, KRSC filter, with the shape rules of
 * infer_conv_shape.  algo: MIQ_ALGO_AUTO (the MFMA implicit GEMM when (c/groups) % 4 == 0 and
 * x, w are 16-byte aligned, else the direct kernel), MIQ_ALGO_IGEMM (MIQ_ERR_UNSUPPORTED
 * where it does not apply) or MIQ_ALGO_DIRECT (the reference CPU loop's order and rounding:
 * cpu_fprop_nhwc's result bit for bit).  The implicit GEMM sums in another order; it agrees
 * with cpu_fprop_nhwc within the reference's own check (abs 1e-4 / rel 1e-3).
 * Replaces launch_fprop_nhwc (/root/reference/src/cuda_kernels.cu:767-823). */
int miq_fprop_nhwc_f32(const float* x, const float* w, float* y, int32_t n, int32_t h, int32_t wdt, int32_t c,
                       int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p, int32_t algo, void* stream);

/* dx = the gradient of the convolution with respect to x, for output gradient dy (NHWC,
 * n x ho x wo x k) and filter w; dx is NHWC n x h x w x c, fully overwritten.  algo:
 * MIQ_ALGO_AUTO (the MFMA implicit GEMM for stride 1, (k/groups) % 4 == 0 and 16-byte aligned
 * dy, else direct), MIQ_ALGO_IGEMM (MIQ_ERR_UNSUPPORTED where it does not apply; agrees with
 * cpu_bprop_nhwc within abs 1e-4 / rel 1e-3) or MIQ_ALGO_DIRECT (the loop order and rounding
 * of cpu_bprop_nhwc: its result bit for bit).
 * Replaces launch_bprop_nhwc (/root/reference/src/cuda_kernels.cu:825-872). */
int miq_bprop_nhwc_f32(const float* dy, const float* w, float* dx, int32_t n, int32_t h, int32_t wdt, int32_t c,
                       int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p, int32_t algo, void* stream);

/* dw = the gradient with respect to the KRSC filter (k x r x s x c/groups, fully overwritten)
 * for input x and output gradient dy.  algo:
 *   MIQ_ALGO_AUTO: the depthwise kernel (c/groups == k/groups == 1, c % 4 == 0, r*s <= 16,
 *     16-byte aligned x and dy), else the MFMA GEMM over pixels; both split the pixels over
 *     workgroups and add the split partial sums in a fixed order, so every call gives the same
 *     bits (as the reference's ordered GEMM does);
 *   MIQ_ALGO_IGEMM: the MFMA GEMM, ordered (MIQ_ERR_UNSUPPORTED where it does not apply);
 *   MIQ_ALGO_ATOMIC: AUTO's kernel with the partial sums added into dw by float atomics: no
 *     workspace, but the bits vary from run to run;
 *   MIQ_ALGO_DIRECT: the loop order and rounding of cpu_grad_nhwc: its result bit for bit.
 * The split kernels agree with cpu_grad_nhwc within abs 1e-4 / rel 1e-3, not bit for bit.
 * The ordered sums need a device workspace: this entry point keeps one per device, allocated
 * (hipMalloc) on first use and grown as the reference's static workspace is, without freeing
 * the outgrown buffer or synchronising; calls that overlap on one device share it and race.
 * Replaces launch_grad_nhwc (/root/reference/src/cuda_kernels.cu:874-937). */
int miq_grad_nhwc_f32(const float* x, const float* dy, float* dw, int32_t n, int32_t h, int32_t wdt, int32_t c,
                      int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p, int32_t algo, void* stream);

/* Bytes of device workspace miq_grad_nhwc_f32_ws needs for this shape and algo (0 when the
 * kernel needs none: DIRECT, ATOMIC, or a single split).  No GPU access.  Has no reference
 * counterpart: it sizes the caller-provided form of launch_grad_nhwc's workspace. */
int miq_grad_nhwc_f32_workspace_size(int32_t n, int32_t h, int32_t wdt, int32_t c, int32_t r, int32_t s, int32_t k,
                                     const miq_conv2d_params* p, int32_t algo, size_t* bytes);

/* miq_grad_nhwc_f32 with a caller-provided device workspace of at least
 * miq_grad_nhwc_f32_workspace_size bytes (it may be NULL when that size is 0); allocates
 * nothing.  Same result bits as miq_grad_nhwc_f32 for the same algo.  The workspace must not
 * be used by another call until this one's work on `stream` has finished.
 * Replaces launch_grad_nhwc (/root/reference/src/cuda_kernels.cu:874-937) with the
 * reference's internal workspace (:155-158, :885-891) passed in instead. */
int miq_grad_nhwc_f32_ws(const float* x, const float* dy, float* dw, int32_t n, int32_t h, int32_t wdt, int32_t c,
                         int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p, int32_t algo, void* workspace,
                         size_t workspace_bytes, void* stream);

/* miq_grad_nhwc_f32 (same algo values, same result bits) without any device allocation: the
 * ordered split partial sums live in a file-scope device array of the library, 32 MiB per
 * device, allocated when the library's device code is loaded on a device (its first kernel
 * launch there, whichever entry point makes it) and held until the process ends.  Shapes whose partial
 * sums need more (miq_grad_nhwc_f32_workspace_size > 33554432 bytes) are rejected with
 * MIQ_ERR_UNSUPPORTED before anything is enqueued.  Calls that overlap on one device (other
 * streams or threads) share the array and race.  No reference counterpart: it exists for
 * callers that cannot allocate (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc). */
int miq_grad_nhwc_f32_noalloc(const float* x, const float* dy, float* dw, int32_t n, int32_t h, int32_t wdt,
                              int32_t c, int32_t r, int32_t s, int32_t k, const miq_conv2d_params* p, int32_t algo,
                              void* stream);

/* ---- blocked (locally connected) fp32 convolution ----------------------------------- */
/* The output grid splits into block_by x block_bx blocks of (ho / block_by) x (wo / block_bx)
 * positions (ho and wo must divide; miq_block_conv_output_shape), each with its own filter:
 * w is [k][block_by][block_bx][r][s][c/groups].  Bias and its gradient are k * block_by *
 * block_bx floats indexed [k][by][bx]; with MIQ_BLOCK_BIAS_SHARED every block uses (and the
 * gradient accumulates into) entry [k][0][0], the other entries of dbias being set to 0.
 * Values of BlockBiasMode (/root/reference/src/conv_types.h:37-40). */
typedef enum miq_block_bias_mode {
  MIQ_BLOCK_BIAS_PER_BLOCK = 0,
  MIQ_BLOCK_BIAS_SHARED = 1
} miq_block_bias_mode;

/* y = the blocked convolution of x (then + bias, one fp32 add after the tap sum, when bias is
 * not NULL).  algo: MIQ_ALGO_AUTO (the MFMA implicit GEMM, one block per workgroup, where
 * miq_fprop_nhwc_f32 would take it; else direct), MIQ_ALGO_IGEMM or MIQ_ALGO_DIRECT (the
 * loop order and rounding of cpu_block_fprop_nhwc, cpu_ref.cpp:232-270: its result bit for
 * bit).  Replaces launch_block_fprop_nhwc (/root/reference/src/cuda_kernels.cu:939-1001). */
int miq_block_fprop_nhwc_f32(const float* x, const float* w, float* y, int32_t n, int32_t h, int32_t wdt, int32_t c,
                             int32_t r, int32_t s, int32_t k, const miq_block_conv2d_params* p, const float* bias,
                             int32_t bias_mode, int32_t algo, void* stream);

/* dx of the blocked convolution (dy n x ho x wo x k; dx fully overwritten).  algo: as
 * miq_bprop_nhwc_f32 (the MFMA form: stride 1, each dx tile reducing over the filter blocks its
 * taps reach); MIQ_ALGO_DIRECT follows cpu_block_bprop_nhwc (cpu_ref.cpp:272-314) bit for bit.
 * Replaces launch_block_bprop_nhwc (/root/reference/src/cuda_kernels.cu:1003-1058). */
int miq_block_bprop_nhwc_f32(const float* dy, const float* w, float* dx, int32_t n, int32_t h, int32_t wdt, int32_t c,
                             int32_t r, int32_t s, int32_t k, const miq_block_conv2d_params* p, int32_t algo,
                             void* stream);

/* dw ([k][by][bx][r][s][c/groups], fully overwritten) of the blocked convolution and, when
 * dbias is not NULL, the bias gradient: the sum of dy over every output position of the block
 * (k * by * bx floats, fully overwritten), as launch_block_grad_nhwc computes it, added in a
 * fixed order so that every call gives the same bits (the reference's CPU form,
 * cpu_block_grad_nhwc, counts only the positions whose (r, s) = (0, 0) tap lies inside the
 * image: the two differ where that tap falls in the padding).  algo: as miq_grad_nhwc_f32;
 * MIQ_ALGO_DIRECT gives cpu_block_grad_nhwc's dw (cpu_ref.cpp:316-369) bit for bit.  Keeps the
 * grow-only per-device workspace of miq_grad_nhwc_f32.
 * Replaces launch_block_grad_nhwc (/root/reference/src/cuda_kernels.cu:1060-1136). */
int miq_block_grad_nhwc_f32(const float* x, const float* dy, float* dw, int32_t n, int32_t h, int32_t wdt, int32_t c,
                            int32_t r, int32_t s, int32_t k, const miq_block_conv2d_params* p, float* dbias,
                            int32_t bias_mode, int32_t algo, void* stream);

/* Kernel families of the fp32 passes (miq_plan_f32). */
typedef enum miq_f32_kernel {
  MIQ_F32_DIRECT = 0,          /* the reference CPU loop's order, one thread per output element (dx: per 4
                                  channels when (c/groups) % 4 == 0 and dx, w are 16-byte aligned) */
  MIQ_F32_IGEMM = 1,           /* fp32 MFMA implicit GEMM, 128 pixels x 64 channels per workgroup */
  MIQ_F32_IGEMM32 = 2,         /* the same with 256 pixels x 32 channels (groups of <= 32 channels) */
  MIQ_F32_DEPTHWISE = 3,       /* depthwise fprop or dx, 4 channels per thread */
  MIQ_F32_BPROP_IGEMM = 4,     /* stride-1 dx as the forward implicit GEMM over dy */
  MIQ_F32_GRAD_IGEMM = 5,      /* dw as a GEMM over pixels split across workgroups */
  MIQ_F32_GRAD_DEPTHWISE = 6   /* depthwise dw, pixel runs per thread */
} miq_f32_kernel;

/* The kernel family an fp32 pass (op 0 fprop, 1 bprop, 2 grad) would run for this problem and
 * algo, with 16-byte aligned tensors; the same validation as the entry point.  No GPU access.
 * No reference counterpart: it names what launch_fprop_nhwc / launch_bprop_nhwc /
 * launch_grad_nhwc run for benchmark tables and tests. */
int miq_plan_f32(int32_t op, int32_t n, int32_t h, int32_t wdt, int32_t c, int32_t r, int32_t s, int32_t k,
                 const miq_conv2d_params* p, int32_t algo, int32_t* kernel);

/* miq_plan_f32 for the blocked passes (miq_block_fprop_nhwc_f32, miq_block_bprop_nhwc_f32,
 * miq_block_grad_nhwc_f32).  No reference counterpart. */
int miq_plan_block_f32(int32_t op, int32_t n, int32_t h, int32_t wdt, int32_t c, int32_t r, int32_t s, int32_t k,
                       const miq_block_conv2d_params* p, int32_t algo, int32_t* kernel);

/* ---- int32 batched matrix product -------------------------------------------------- */
/* C[b] = op(A[b]) * op(B[b]) for b < batch, with int32 wrap-around (mod 2^32) products and
 * sums, exact for every int32 input.  Row-major, batch strides M*K, K*N and M*N:
 *   A[b] is M x K, or stored K x M when trans_a != 0;
 *   B[b] is K x N, or stored N x K when trans_b != 0;
 *   C[b] is M x N, fully overwritten (K == 0 writes zeros).
 * Extents must be >= 0; batch, M or N == 0 enqueues nothing. */

/* The stream-ordered, status-returning form of bmm_matmul_i32. */
int miq_bmm_i32(const int32_t* A, const int32_t* B, int32_t* C, int32_t batch, int32_t M, int32_t N,
                int32_t K, int32_t trans_a, int32_t trans_b, void* stream);

/* Replaces bmm_matmul_i32 (/root/reference/bmm.cu:298-322, declared bmm.h:69-73): same
 * symbol, arguments and meaning, on the default stream.  Like the reference it returns
 * nothing; a rejected call enqueues nothing and leaves its reason in
 * miq_last_error_message(). */
void bmm_matmul_i32(const int32_t* A, const int32_t* B, int32_t* C, int batch, int M, int N, int K,
                    int trans_a, int trans_b);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif /* MIQ_QCONV_H_ */
