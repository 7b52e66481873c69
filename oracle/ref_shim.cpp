// ref_shim.cpp - extern "C" access to the reference's own CPU path, compiled from the
// reference's sources where they lie (see oracle/Makefile; output in oracle/_ref/).
//
// TEST INFRASTRUCTURE ONLY: used by tests/ (golden vectors, oracle pinning) and by
// bench.py's cpu_baseline leg.  Builds the reference's TensorNHWC / FilterKRSC /
// BlockFilterKByBxRSC from flat arrays, calls cpu_fprop_nhwc_qi32<Tin> /
// cpu_block_fprop_nhwc_qi32<Tin> (/root/reference/src/conv_types.h:255-285 ->
// cpu_ref.cpp:36-112, :371-401), cpu_fprop_nhwc / cpu_bprop_nhwc / cpu_grad_nhwc
// (cpu_ref.cpp:116-230) and verify_tensors
// (src/verify.cpp:7-36).

#include <chrono>
#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "conv_types.h"

namespace {

thread_local std::string g_err;

using nnalgebra::DataType;
template <DataType T>
using QP = nnalgebra::QuantizationParameters<T>;

Conv2DParams to_params(const int32_t conv[7]) {
  Conv2DParams p;
  p.pad_h = conv[0]; p.pad_w = conv[1];
  p.stride_h = conv[2]; p.stride_w = conv[3];
  p.dilation_h = conv[4]; p.dilation_w = conv[5];
  p.groups = conv[6];
  return p;
}

template <DataType T>
std::vector<QP<T>> input_qparams(int n, const int32_t* zp) {
  std::vector<QP<T>> qp(static_cast<size_t>(n));
  for (int i = 0; i < n; ++i) qp[static_cast<size_t>(i)].zero_point = static_cast<decltype(qp[0].zero_point)>(zp[i]);
  return qp;
}

template <DataType T>
int run(const float* x, int n, int h, int w, int c, const float* wt, int r, int s, int k, const int32_t conv[7],
        const int32_t* in_zp, int32_t f_zp, int by, int bx, int32_t* y, double* seconds) {
  try {
    const Conv2DParams p = to_params(conv);
    TensorNHWC xt(n, h, w, c);
    std::memcpy(xt.ptr(), x, xt.elements() * sizeof(float));
    const auto iq = input_qparams<T>(n, in_zp);
    QP<T> fq;
    fq.zero_point = static_cast<decltype(fq.zero_point)>(f_zp);
    TensorNHWCI32 yt;
    const int cg = (p.groups > 0) ? c / p.groups : 0;
    const auto t0 = std::chrono::steady_clock::now();
    if (by > 0 && bx > 0) {
      BlockConv2DParams bp;
      bp.conv = p;
      bp.block_by = by;
      bp.block_bx = bx;
      BlockFilterKByBxRSC ft(k, by, bx, r, s, cg);
      std::memcpy(ft.ptr(), wt, ft.elements() * sizeof(float));
      const auto t1 = std::chrono::steady_clock::now();
      cpu_block_fprop_nhwc_qi32<T>(xt, ft, bp, yt, iq.data(), &fq);
      if (seconds) *seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t1).count();
    } else {
      FilterKRSC ft(r, s, cg, k);
      std::memcpy(ft.ptr(), wt, ft.elements() * sizeof(float));
      const auto t1 = std::chrono::steady_clock::now();
      cpu_fprop_nhwc_qi32<T>(xt, ft, p, yt, iq.data(), &fq);
      if (seconds) *seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t1).count();
    }
    (void)t0;
    std::memcpy(y, yt.ptr(), yt.elements() * sizeof(int32_t));
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

}  // namespace

extern "C" {

const char* ref_last_error(void) { return g_err.c_str(); }

// kind 0: LinQuantU8, 1: LinQuantS5.  by = bx = 0: regular filter.  `seconds` (nullable)
// receives the wall time of the reference call alone.
int ref_fprop_qi32(int kind, const float* x, int n, int h, int w, int c, const float* wt, int r, int s, int k,
                   const int32_t conv[7], const int32_t* in_zp, int32_t f_zp, int by, int bx, int32_t* y,
                   double* seconds) {
  if (kind == 0) return run<DataType::LinQuantU8>(x, n, h, w, c, wt, r, s, k, conv, in_zp, f_zp, by, bx, y, seconds);
  return run<DataType::LinQuantS5>(x, n, h, w, c, wt, r, s, k, conv, in_zp, f_zp, by, bx, y, seconds);
}

// cpu_fprop_nhwc (cpu_ref.cpp:116-146) on flat NHWC / KRSC arrays; `seconds` (nullable)
// receives the wall time of the reference call alone.
int ref_fprop_f32(const float* x, int n, int h, int w, int c, const float* wt, int r, int s, int k,
                  const int32_t conv[7], float* y, double* seconds) {
  try {
    const Conv2DParams p = to_params(conv);
    TensorNHWC xt(n, h, w, c);
    std::memcpy(xt.ptr(), x, xt.elements() * sizeof(float));
    const int cg = (p.groups > 0) ? c / p.groups : 0;
    FilterKRSC ft(r, s, cg, k);
    std::memcpy(ft.ptr(), wt, ft.elements() * sizeof(float));
    TensorNHWC yt;
    const auto t1 = std::chrono::steady_clock::now();
    cpu_fprop_nhwc(xt, ft, p, yt);
    if (seconds) *seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t1).count();
    std::memcpy(y, yt.ptr(), yt.elements() * sizeof(float));
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

// cpu_bprop_nhwc (cpu_ref.cpp:150-190) / cpu_grad_nhwc (:192-230) on flat arrays: `a` is dy
// (op 0, result dx, n x h x w x c) or x (op 1, result dw, KRSC), `b` the filter (op 0) or dy
// (op 1).
int ref_backward_f32(int op, const float* a, const float* b, int n, int h, int w, int c, int r, int s, int k,
                     const int32_t conv[7], float* out, double* seconds) {
  try {
    const Conv2DParams p = to_params(conv);
    const int cg = (p.groups > 0) ? c / p.groups : 0;
    TensorNHWC xs(n, h, w, c);
    FilterKRSC fs(r, s, cg, k);
    const ConvShape sh = infer_conv_shape(xs, fs, p);
    TensorNHWC dy(n, sh.ho, sh.wo, k);
    const auto t1 = std::chrono::steady_clock::now();
    if (op == 0) {
      std::memcpy(dy.ptr(), a, dy.elements() * sizeof(float));
      std::memcpy(fs.ptr(), b, fs.elements() * sizeof(float));
      TensorNHWC dx(n, h, w, c);
      cpu_bprop_nhwc(dy, fs, p, dx);
      std::memcpy(out, dx.ptr(), dx.elements() * sizeof(float));
    } else {
      std::memcpy(xs.ptr(), a, xs.elements() * sizeof(float));
      std::memcpy(dy.ptr(), b, dy.elements() * sizeof(float));
      FilterKRSC dw(r, s, cg, k);
      cpu_grad_nhwc(xs, dy, p, dw);
      std::memcpy(out, dw.ptr(), dw.elements() * sizeof(float));
    }
    if (seconds) *seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t1).count();
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

// cpu_block_fprop_nhwc (cpu_ref.cpp:232-270, op 0: a = x, b = w, out = y, bias nullable),
// cpu_block_bprop_nhwc (:272-314, op 1: a = dy, b = w, out = dx) and cpu_block_grad_nhwc
// (:316-369, op 2: a = x, b = dy, out = dw, `bias` receives dbias when given) on flat arrays;
// the filter is [k][by][bx][r][s][c/groups], bias / dbias k*by*bx floats, bias_mode 0
// (PerBlock) or 1 (Shared).
int ref_block_f32(int op, const float* a, const float* b, int n, int h, int w, int c, int r, int s, int k,
                  const int32_t conv[7], int by, int bx, float* bias, int bias_mode, float* out, double* seconds) {
  try {
    BlockConv2DParams p;
    p.conv = to_params(conv);
    p.block_by = by;
    p.block_bx = bx;
    const int cg = (p.conv.groups > 0) ? c / p.conv.groups : 0;
    const BlockBiasMode mode = bias_mode == 0 ? BlockBiasMode::PerBlock : BlockBiasMode::Shared;
    TensorNHWC xs(n, h, w, c);
    if (by <= 0 || bx <= 0) throw std::runtime_error("block_by and block_bx must be > 0");
    BlockFilterKByBxRSC fs(k, by, bx, r, s, cg);
    const BlockConvShape sh = infer_block_conv_shape(xs, fs, p);
    const size_t dy_elems = static_cast<size_t>(n) * sh.base.ho * sh.base.wo * k;
    const auto t1 = std::chrono::steady_clock::now();
    if (op == 0) {
      std::memcpy(xs.ptr(), a, xs.elements() * sizeof(float));
      std::memcpy(fs.ptr(), b, fs.elements() * sizeof(float));
      TensorNHWC y;
      cpu_block_fprop_nhwc(xs, fs, p, y, bias, mode);
      std::memcpy(out, y.ptr(), y.elements() * sizeof(float));
    } else if (op == 1) {
      TensorNHWC dy(n, sh.base.ho, sh.base.wo, k);
      std::memcpy(dy.ptr(), a, dy_elems * sizeof(float));
      std::memcpy(fs.ptr(), b, fs.elements() * sizeof(float));
      cpu_block_bprop_nhwc(dy, fs, p, xs);
      std::memcpy(out, xs.ptr(), xs.elements() * sizeof(float));
    } else {
      TensorNHWC dy(n, sh.base.ho, sh.base.wo, k);
      std::memcpy(xs.ptr(), a, xs.elements() * sizeof(float));
      std::memcpy(dy.ptr(), b, dy_elems * sizeof(float));
      cpu_block_grad_nhwc(xs, dy, p, fs, bias, mode);
      std::memcpy(out, fs.ptr(), fs.elements() * sizeof(float));
    }
    if (seconds) *seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t1).count();
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

int ref_verify_tensors(const float* ref, const float* got, size_t count, float abs_eps, float rel_eps,
                       float* max_abs, float* max_rel, size_t* abs_idx, size_t* rel_idx, int* passed) {
  try {
    const std::vector<float> a(ref, ref + count), b(got, got + count);
    const VerifyResult v = verify_tensors(a, b, abs_eps, rel_eps);
    *max_abs = v.max_abs_err; *max_rel = v.max_rel_err;
    *abs_idx = v.max_abs_idx; *rel_idx = v.max_rel_idx;
    *passed = v.passed ? 1 : 0;
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

}  // extern "C"

extern "C" {

// infer_conv_shape of the reference header (conv_types.h:125-146) on a tensor / filter of
// the given extents: 0 and (ho, wo), or -1 and the exception text in ref_last_error().
int ref_infer_conv_shape(int n, int h, int w, int c, int r, int s, int k, const int32_t conv[7], int* ho, int* wo) {
  try {
    const Conv2DParams p = to_params(conv);
    TensorNHWC x;  // extents only: no allocation
    x.n = n; x.h = h; x.w = w; x.c = c;
    FilterKRSC f;
    f.r = r; f.s = s; f.k = k;
    f.cin_per_group = (p.groups > 0) ? c / p.groups : 0;
    const ConvShape sh = infer_conv_shape(x, f, p);
    *ho = sh.ho;
    *wo = sh.wo;
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

}  // extern "C"
