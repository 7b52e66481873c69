/*
 * qconv_oracle.c - CPU restatement of the reference's quantized NHWC convolution.
 *
 * TEST INFRASTRUCTURE ONLY: the checker of the HIP library (see qconv_oracle.h).  Not
 * part of the product; nothing in my_own_cnn_amd/ links or calls it.
 *
 * Pinning (the checks that hold this restatement to the reference, in tests/):
 *   orc_conv_qi32        golden vectors from the reference's own cpu_ref.cpp compiled in
 *                        this repository (oracle/_ref), the four quant_conv_test cases,
 *                        float64 convolution, brute force and conv identities.
 *   orc_conv_i8_acc      the same, plus C1 in full and C2-C5 hashes from oracle/_ref.
 *   orc_requant_i8 /     no reference counterpart (the reference has no requantization):
 *   orc_dequant_f32      hand-computed known answers and float64 bounds.
 *   orc_fill_*           fixed known outputs of splitmix64.
 *   orc_conv_f32,        the reference's own cpu_fprop_nhwc / cpu_bprop_nhwc / cpu_grad_nhwc
 *   orc_bprop_f32,       compiled in oracle/_ref (bit for bit: same loop orders and fp32
 *   orc_grad_f32         operations); float64 torch convolution and its autograd gradients.
 *   orc_bmm_i32          unsigned 64-bit numpy products reduced mod 2^32, brute force on
 *                        tiny inputs, wrap-around known answers (INT_MIN, INT_MAX), and at
 *                        the reference's call site (cuda_kernels.cu:1381: im2col columns x
 *                        packed filter, trans_b) the convolution accumulators of
 *                        orc_conv_qi32 and of oracle/_ref.
 */
#include "qconv_oracle.h"

#include <math.h>
#include <stddef.h>
#include <stdint.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- synthetic data -------------------------------------------------------------- */

/* splitmix64 (Steele, Lea, Flood 2014): state_i = seed + (i+1) * 0x9E3779B97F4A7C15,
 * output = the mixing finaliser of state_i. */
uint64_t orc_splitmix64(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1u) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* lo + floor(hi32(u) * (hi - lo + 1) / 2^32) */
void orc_fill_i8_uniform(int8_t* out, int64_t count, uint64_t seed, int32_t lo, int32_t hi) {
  const uint64_t range = (uint64_t)((int64_t)hi - lo + 1);
  for (int64_t i = 0; i < count; ++i) {
    const uint64_t u = orc_splitmix64(seed, (uint64_t)i);
    out[i] = (int8_t)(lo + (int32_t)(((u >> 32) * range) >> 32));
  }
}

/* post-ReLU activations: 0 when the top bit is clear, else 1 + floor(lo32(u) * 127 / 2^32) */
void orc_fill_i8_relu_half(int8_t* out, int64_t count, uint64_t seed) {
  for (int64_t i = 0; i < count; ++i) {
    const uint64_t u = orc_splitmix64(seed, (uint64_t)i);
    out[i] = (u >> 63) ? (int8_t)(1 + (int32_t)(((u & 0xffffffffull) * 127u) >> 32)) : (int8_t)0;
  }
}

void orc_fill_i32_uniform(int32_t* out, int64_t count, uint64_t seed, int32_t lo, int32_t hi) {
  const uint64_t range = (uint64_t)((int64_t)hi - lo + 1);
  for (int64_t i = 0; i < count; ++i) {
    const uint64_t u = orc_splitmix64(seed, (uint64_t)i);
    out[i] = (int32_t)((int64_t)lo + (int64_t)(((u >> 32) * range) >> 32));
  }
}

/* lo + f * (hi - lo) in single precision, f = top 24 bits of u / 2^24 (exact in fp32) */
void orc_fill_f32_uniform(float* out, int64_t count, uint64_t seed, float lo, float hi) {
  const float span = hi - lo;
  for (int64_t i = 0; i < count; ++i) {
    const uint64_t u = orc_splitmix64(seed, (uint64_t)i);
    const float f = (float)(u >> 40) * 0x1p-24f;
    const float t = f * span;
    out[i] = lo + t;
  }
}

/* ---- shape ------------------------------------------------------------------------- */

/* Follows infer_conv_shape (/root/reference/src/conv_types.h:125-146). */
int orc_conv_output_shape(int32_t n, int32_t h, int32_t w, int32_t c, int32_t r, int32_t s, int32_t k,
                          const int32_t conv[7], int32_t* ho, int32_t* wo) {
  (void)n;
  const int32_t groups = conv[6];
  if (groups <= 0 || c % groups != 0 || k % groups != 0) return -1;
  const int64_t rows = (int64_t)h + 2 * (int64_t)conv[0] - (int64_t)conv[4] * (r - 1) - 1;
  const int64_t cols = (int64_t)w + 2 * (int64_t)conv[1] - (int64_t)conv[5] * (s - 1) - 1;
  if (rows < 0 || cols < 0) return -1;
  if (conv[2] <= 0 || conv[3] <= 0) return -1;
  *ho = (int32_t)(rows / conv[2] + 1);
  *wo = (int32_t)(cols / conv[3] + 1);
  if (*ho <= 0 || *wo <= 0) return -1;
  return 0;
}

/* ---- int32 accumulation ------------------------------------------------------------ */

/* Follows cpu_fprop_nhwc_qi32_impl and cpu_block_fprop_nhwc_qi32_impl
 * (/root/reference/src/cpu_ref.cpp:36-112) with the helpers they call
 * (centered_input_value :11-17, centered_weight_value :19-25,
 * centered_block_weight_value :27-34, output_block_index :7-9): loop order
 * n, ho, wo, g, ko, r, s, ci; codes truncated to int32; taps outside the input skipped;
 * the sample's zero point subtracted from inputs and the filter's from weights;
 * output channel g*Kg + ko.  Sums use unsigned (wrap-around) arithmetic, which equals the
 * reference's int32 result whenever the reference's is defined. */
int orc_conv_qi32(const float* x, int32_t n, int32_t h, int32_t w, int32_t c, const float* wt, int32_t r,
                  int32_t s, int32_t k, const int32_t conv[7], const int32_t* in_zp, int32_t f_zp, int32_t by,
                  int32_t bx, int32_t* y) {
  int32_t ho_n, wo_n;
  if (orc_conv_output_shape(n, h, w, c, r, s, k, conv, &ho_n, &wo_n) != 0) return -1;
  const int blocked = (by > 0 && bx > 0);
  if (blocked && (ho_n % by != 0 || wo_n % bx != 0)) return -1;
  const int32_t ph = conv[0], pw = conv[1], sh = conv[2], sw = conv[3], dh = conv[4], dw = conv[5], g_n = conv[6];
  const int32_t cg = c / g_n, kg = k / g_n;
  const int32_t bho = blocked ? ho_n / by : 1, bwo = blocked ? wo_n / bx : 1;
  for (int32_t ni = 0; ni < n; ++ni) {
    for (int32_t ho = 0; ho < ho_n; ++ho) {
      const int32_t byi = blocked ? ho / bho : 0;
      for (int32_t wo = 0; wo < wo_n; ++wo) {
        const int32_t bxi = blocked ? wo / bwo : 0;
        for (int32_t g = 0; g < g_n; ++g) {
          for (int32_t ko = 0; ko < kg; ++ko) {
            const int32_t kk = g * kg + ko;
            uint32_t acc = 0;
            for (int32_t rr = 0; rr < r; ++rr) {
              const int32_t hi = ho * sh - ph + rr * dh;
              if (hi < 0 || hi >= h) continue;
              for (int32_t ss = 0; ss < s; ++ss) {
                const int32_t wi = wo * sw - pw + ss * dw;
                if (wi < 0 || wi >= w) continue;
                for (int32_t ci = 0; ci < cg; ++ci) {
                  const size_t xi = (((size_t)ni * h + hi) * w + wi) * c + (size_t)g * cg + ci;
                  size_t wj;
                  if (blocked) {
                    wj = (((((size_t)kk * by + byi) * bx + bxi) * r + rr) * s + ss) * cg + ci;
                  } else {
                    wj = (((size_t)kk * r + rr) * s + ss) * cg + ci;
                  }
                  const int32_t xv = (int32_t)x[xi] - in_zp[ni];
                  const int32_t wv = (int32_t)wt[wj] - f_zp;
                  acc += (uint32_t)xv * (uint32_t)wv;
                }
              }
            }
            y[(((size_t)ni * ho_n + ho) * wo_n + wo) * k + kk] = (int32_t)acc;
          }
        }
      }
    }
  }
  return 0;
}

/* The same accumulation (cpu_ref.cpp:36-72) for int8 codes with zero points 0; output
 * rows (n, ho) are independent and are spread over OpenMP threads. */
int orc_conv_i8_acc(const int8_t* x, int32_t n, int32_t h, int32_t w, int32_t c, const int8_t* wt, int32_t r,
                    int32_t s, int32_t k, const int32_t conv[7], int32_t* y, int32_t nthreads) {
  int32_t ho_n, wo_n;
  if (orc_conv_output_shape(n, h, w, c, r, s, k, conv, &ho_n, &wo_n) != 0) return -1;
  const int32_t ph = conv[0], pw = conv[1], sh = conv[2], sw = conv[3], dh = conv[4], dw = conv[5], g_n = conv[6];
  const int32_t cg = c / g_n, kg = k / g_n;
  const int64_t nrows = (int64_t)n * ho_n;
#ifdef _OPENMP
  const int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#else
  (void)nthreads;
#endif
  for (int64_t row = 0; row < nrows; ++row) {
    const int32_t ni = (int32_t)(row / ho_n);
    const int32_t ho = (int32_t)(row % ho_n);
    for (int32_t wo = 0; wo < wo_n; ++wo) {
      for (int32_t g = 0; g < g_n; ++g) {
        for (int32_t ko = 0; ko < kg; ++ko) {
          const int32_t kk = g * kg + ko;
          uint32_t acc = 0;
          for (int32_t rr = 0; rr < r; ++rr) {
            const int32_t hi = ho * sh - ph + rr * dh;
            if (hi < 0 || hi >= h) continue;
            for (int32_t ss = 0; ss < s; ++ss) {
              const int32_t wi = wo * sw - pw + ss * dw;
              if (wi < 0 || wi >= w) continue;
              const int8_t* xp = x + (((size_t)ni * h + hi) * w + wi) * c + (size_t)g * cg;
              const int8_t* wp = wt + (((size_t)kk * r + rr) * s + ss) * cg;
              int32_t dot = 0; /* |dot| <= cg * 2^14: exact for any cg < 2^17 */
              for (int32_t ci = 0; ci < cg; ++ci) dot += (int32_t)xp[ci] * (int32_t)wp[ci];
              acc += (uint32_t)dot;
            }
          }
          y[(((size_t)ni * ho_n + ho) * wo_n + wo) * k + kk] = (int32_t)acc;
        }
      }
    }
  }
  return 0;
}

/* ---- requantization (no reference counterpart) ------------------------------------- */

/* a = in_scale / out_scale; m = a * w_scale[k]; v = (float)(acc + bias[k]) * m;
 * q = rint(v) with ties to even; q < lo (or NaN) -> lo; q > 127 -> 127. */
void orc_requant_i8(const int32_t* acc, int64_t npix, int32_t k, const int32_t* bias, const float* w_scale,
                    float in_scale, float out_scale, int32_t relu, int8_t* y) {
  const float a = in_scale / out_scale;
  const float lo = relu ? 0.0f : -128.0f;
  for (int64_t p = 0; p < npix; ++p) {
    for (int32_t kk = 0; kk < k; ++kk) {
      const size_t i = (size_t)p * k + kk;
      const float m = a * w_scale[kk];
      const int32_t t = (int32_t)((uint32_t)acc[i] + (uint32_t)(bias ? bias[kk] : 0));
      const float v = (float)t * m;
      float q = rintf(v); /* default rounding mode: to nearest, ties to even */
      q = (q >= lo) ? q : lo;
      q = (q > 127.0f) ? 127.0f : q;
      y[i] = (int8_t)(int32_t)q;
    }
  }
}

/* v = (float)(acc + bias[k]) * m; with relu, v <= 0 or NaN becomes +0. */
void orc_dequant_f32(const int32_t* acc, int64_t npix, int32_t k, const int32_t* bias, const float* w_scale,
                     float in_scale, float out_scale, int32_t relu, float* y) {
  const float a = in_scale / out_scale;
  for (int64_t p = 0; p < npix; ++p) {
    for (int32_t kk = 0; kk < k; ++kk) {
      const size_t i = (size_t)p * k + kk;
      const float m = a * w_scale[kk];
      const int32_t t = (int32_t)((uint32_t)acc[i] + (uint32_t)(bias ? bias[kk] : 0));
      float v = (float)t * m;
      if (relu) v = (v > 0.0f) ? v : 0.0f;
      y[i] = v;
    }
  }
}

/* ---- int32 batched matrix product --------------------------------------------------- */

/* bmm_matmul_i32 (/root/reference/bmm.cu:298-322, kernel bmm.cu:155-246): for each batch
 * entry b, C[b][m][n] = sum_k op(A)[m][k] * op(B)[k][n] with A[b] at offset b*M*K stored
 * M x K (K x M when trans_a, read as A[k*M + m], bmm.cu:185-191), B[b] at b*K*N stored K x N
 * (N x K when trans_b, read as B[n*K + k], bmm.cu:200-206), C[b] at b*M*N.  The reference
 * accumulates in int32 on the GPU, where signed multiply and add wrap modulo 2^32; the
 * restatement computes in uint32, whose arithmetic is defined to wrap the same way.  Rows
 * (b, m) are spread over `nthreads` OpenMP threads (<= 0: the OpenMP default). */
void orc_bmm_i32(const int32_t* A, const int32_t* B, int32_t* C, int32_t batch, int32_t M, int32_t N, int32_t K,
                 int32_t trans_a, int32_t trans_b, int32_t nthreads) {
  const int64_t rows = (int64_t)batch * M;
#ifdef _OPENMP
  const int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 16) num_threads(nt)
#else
  (void)nthreads;
#endif
  for (int64_t row = 0; row < rows; ++row) {
    const int64_t b = row / M;
    const int64_t m = row % M;
    const int32_t* Ab = A + b * M * K;
    const int32_t* Bb = B + b * K * N;
    uint32_t* Cr = (uint32_t*)C + b * M * N + m * N;
    for (int32_t n = 0; n < N; ++n) Cr[n] = 0;
    for (int32_t k = 0; k < K; ++k) {
      const uint32_t a = (uint32_t)(trans_a ? Ab[(int64_t)k * M + m] : Ab[m * K + k]);
      if (trans_b) {
        for (int32_t n = 0; n < N; ++n) Cr[n] += a * (uint32_t)Bb[(int64_t)n * K + k];
      } else {
        const int32_t* Bk = Bb + (int64_t)k * N;
        for (int32_t n = 0; n < N; ++n) Cr[n] += a * (uint32_t)Bk[n];
      }
    }
  }
}

/* ---- fp32 convolution ----------------------------------------------------------------- */

/* cpu_fprop_nhwc (/root/reference/src/cpu_ref.cpp:116-146): for each output (n, ho, wo, g, ko)
 * in that loop order, acc = 0.0f and then acc += x * w over r, s, ci (in-bounds taps only),
 * each product and sum one fp32 operation (the library is compiled -ffp-contract=off).
 * Returns 0, or -1 on a shape orc_conv_output_shape rejects. */
int orc_conv_f32(const float* x, int32_t n, int32_t h, int32_t w, int32_t c, const float* wt, int32_t r, int32_t s,
                 int32_t k, const int32_t conv[7], float* y, int32_t nthreads) {
  int32_t ho_n, wo_n;
  if (orc_conv_output_shape(n, h, w, c, r, s, k, conv, &ho_n, &wo_n) != 0) return -1;
  const int32_t ph = conv[0], pw = conv[1], sh = conv[2], sw = conv[3], dh = conv[4], dw = conv[5], g_n = conv[6];
  const int32_t cg = c / g_n, kg = k / g_n;
  const int64_t nrows = (int64_t)n * ho_n;
#ifdef _OPENMP
  const int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#else
  (void)nthreads;
#endif
  for (int64_t row = 0; row < nrows; ++row) {
    const int32_t ni = (int32_t)(row / ho_n);
    const int32_t ho = (int32_t)(row % ho_n);
    for (int32_t wo = 0; wo < wo_n; ++wo) {
      for (int32_t g = 0; g < g_n; ++g) {
        for (int32_t ko = 0; ko < kg; ++ko) {
          float acc = 0.0f;
          for (int32_t rr = 0; rr < r; ++rr) {
            const int32_t hi = ho * sh - ph + rr * dh;
            if (hi < 0 || hi >= h) continue;
            for (int32_t ss = 0; ss < s; ++ss) {
              const int32_t wi = wo * sw - pw + ss * dw;
              if (wi < 0 || wi >= w) continue;
              const float* xp = x + (((size_t)ni * h + hi) * w + wi) * c + (size_t)g * cg;
              const float* wp = wt + ((((size_t)g * kg + ko) * r + rr) * s + ss) * cg;
              for (int32_t ci = 0; ci < cg; ++ci) acc += xp[ci] * wp[ci];
            }
          }
          y[(((size_t)ni * ho_n + ho) * wo_n + wo) * k + (size_t)g * kg + ko] = acc;
        }
      }
    }
  }
  return 0;
}

/* cpu_bprop_nhwc (cpu_ref.cpp:150-190): for each dx element (n, hi, wi, g, ci) in that order,
 * acc = 0.0f, then over taps r, s whose ho = (hi + ph - r dh) / sh is whole and in range
 * (likewise wo), acc += dy[n, ho, wo, g Kg + ko] * w[g Kg + ko, r, s, ci] over ko. */
int orc_bprop_f32(const float* dy, int32_t n, int32_t h, int32_t w, int32_t c, const float* wt, int32_t r, int32_t s,
                  int32_t k, const int32_t conv[7], float* dx, int32_t nthreads) {
  int32_t ho_n, wo_n;
  if (orc_conv_output_shape(n, h, w, c, r, s, k, conv, &ho_n, &wo_n) != 0) return -1;
  const int32_t ph = conv[0], pw = conv[1], sh = conv[2], sw = conv[3], dh = conv[4], dw = conv[5], g_n = conv[6];
  const int32_t cg = c / g_n, kg = k / g_n;
  const int64_t nrows = (int64_t)n * h;
#ifdef _OPENMP
  const int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#else
  (void)nthreads;
#endif
  for (int64_t row = 0; row < nrows; ++row) {
    const int32_t ni = (int32_t)(row / h);
    const int32_t hi = (int32_t)(row % h);
    for (int32_t wi = 0; wi < w; ++wi) {
      for (int32_t g = 0; g < g_n; ++g) {
        for (int32_t ci = 0; ci < cg; ++ci) {
          float acc = 0.0f;
          for (int32_t rr = 0; rr < r; ++rr) {
            const int32_t hn = hi + ph - rr * dh;
            if (hn < 0 || hn % sh != 0) continue;
            const int32_t ho = hn / sh;
            if (ho >= ho_n) continue;
            for (int32_t ss = 0; ss < s; ++ss) {
              const int32_t wn = wi + pw - ss * dw;
              if (wn < 0 || wn % sw != 0) continue;
              const int32_t wo = wn / sw;
              if (wo >= wo_n) continue;
              for (int32_t ko = 0; ko < kg; ++ko) {
                const float dyv = dy[(((size_t)ni * ho_n + ho) * wo_n + wo) * k + (size_t)g * kg + ko];
                const float wv = wt[((((size_t)g * kg + ko) * r + rr) * s + ss) * cg + ci];
                acc += dyv * wv;
              }
            }
          }
          dx[(((size_t)ni * h + hi) * w + wi) * c + (size_t)g * cg + ci] = acc;
        }
      }
    }
  }
  return 0;
}

/* cpu_grad_nhwc (cpu_ref.cpp:192-230): for each dw element (r, s, g, ci, ko) in that order,
 * acc = 0.0f, then acc += x[n, hi, wi, g Cg + ci] * dy[n, ho, wo, g Kg + ko] over n, ho, wo
 * (in-bounds taps); dw is KRSC. */
int orc_grad_f32(const float* x, int32_t n, int32_t h, int32_t w, int32_t c, const float* dy, int32_t r, int32_t s,
                 int32_t k, const int32_t conv[7], float* dwt, int32_t nthreads) {
  int32_t ho_n, wo_n;
  if (orc_conv_output_shape(n, h, w, c, r, s, k, conv, &ho_n, &wo_n) != 0) return -1;
  const int32_t ph = conv[0], pw = conv[1], sh = conv[2], sw = conv[3], dh = conv[4], dw = conv[5], g_n = conv[6];
  const int32_t cg = c / g_n, kg = k / g_n;
  const int64_t nel = (int64_t)k * r * s * cg;
#ifdef _OPENMP
  const int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 16) num_threads(nt)
#else
  (void)nthreads;
#endif
  for (int64_t e = 0; e < nel; ++e) {
    const int32_t ci = (int32_t)(e % cg);
    const int32_t ss = (int32_t)((e / cg) % s);
    const int32_t rr = (int32_t)((e / ((int64_t)cg * s)) % r);
    const int32_t kk = (int32_t)(e / ((int64_t)cg * s * r));
    const int32_t g = kk / kg;
    float acc = 0.0f;
    for (int32_t ni = 0; ni < n; ++ni) {
      for (int32_t ho = 0; ho < ho_n; ++ho) {
        const int32_t hi = ho * sh - ph + rr * dh;
        if (hi < 0 || hi >= h) continue;
        for (int32_t wo = 0; wo < wo_n; ++wo) {
          const int32_t wi = wo * sw - pw + ss * dw;
          if (wi < 0 || wi >= w) continue;
          const float xv = x[(((size_t)ni * h + hi) * w + wi) * c + (size_t)g * cg + ci];
          const float dyv = dy[(((size_t)ni * ho_n + ho) * wo_n + wo) * k + kk];
          acc += xv * dyv;
        }
      }
    }
    dwt[e] = acc;
  }
  return 0;
}

/* ---- blocked fp32 convolution ---------------------------------------------------------- */

/* The blocked shape rules of infer_block_conv_shape (/root/reference/src/conv_types.h:148-169):
 * by, bx > 0 and the output extent divisible by the block grid; bho x bwo output positions
 * per block.  Returns 0, or -1 where the reference throws. */
static int block_shape(int32_t n, int32_t h, int32_t w, int32_t c, int32_t r, int32_t s, int32_t k,
                       const int32_t conv[7], int32_t by, int32_t bx, int32_t* ho_n, int32_t* wo_n, int32_t* bho,
                       int32_t* bwo) {
  if (by <= 0 || bx <= 0) return -1;
  if (orc_conv_output_shape(n, h, w, c, r, s, k, conv, ho_n, wo_n) != 0) return -1;
  if (*ho_n % by != 0 || *wo_n % bx != 0) return -1;
  *bho = *ho_n / by;
  *bwo = *wo_n / bx;
  return 0;
}

/* idx_block_bias (conv_types.h:184-188): mode 0 (PerBlock) indexes [k][by][bx], mode 1
 * (Shared) the block (0, 0) entry of channel k. */
static size_t block_bias_index(int32_t kk, int32_t byi, int32_t bxi, int32_t by, int32_t bx, int32_t mode) {
  const int32_t yi = mode == 0 ? byi : 0, xi = mode == 0 ? bxi : 0;
  return ((size_t)kk * by + yi) * bx + xi;
}

/* cpu_block_fprop_nhwc (cpu_ref.cpp:232-270): as cpu_fprop_nhwc, with output position
 * (ho, wo) in block (ho / bho, wo / bwo) taking its filter from w[k][by][bx][r][s][ci]
 * ([K, By, Bx, R, S, C/groups]); after the tap sum, acc += bias[block_bias_index] where bias
 * is given. */
int orc_block_conv_f32(const float* x, int32_t n, int32_t h, int32_t w, int32_t c, const float* wt, int32_t r,
                       int32_t s, int32_t k, const int32_t conv[7], int32_t by, int32_t bx, const float* bias,
                       int32_t bias_mode, float* y, int32_t nthreads) {
  int32_t ho_n, wo_n, bho, bwo;
  if (block_shape(n, h, w, c, r, s, k, conv, by, bx, &ho_n, &wo_n, &bho, &bwo) != 0) return -1;
  const int32_t ph = conv[0], pw = conv[1], sh = conv[2], sw = conv[3], dh = conv[4], dw = conv[5], g_n = conv[6];
  const int32_t cg = c / g_n, kg = k / g_n;
  const int64_t nrows = (int64_t)n * ho_n;
#ifdef _OPENMP
  const int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#else
  (void)nthreads;
#endif
  for (int64_t row = 0; row < nrows; ++row) {
    const int32_t ni = (int32_t)(row / ho_n);
    const int32_t ho = (int32_t)(row % ho_n);
    const int32_t byi = ho / bho;
    for (int32_t wo = 0; wo < wo_n; ++wo) {
      const int32_t bxi = wo / bwo;
      for (int32_t g = 0; g < g_n; ++g) {
        for (int32_t ko = 0; ko < kg; ++ko) {
          const int32_t kk = g * kg + ko;
          float acc = 0.0f;
          for (int32_t rr = 0; rr < r; ++rr) {
            const int32_t hi = ho * sh - ph + rr * dh;
            if (hi < 0 || hi >= h) continue;
            for (int32_t ss = 0; ss < s; ++ss) {
              const int32_t wi = wo * sw - pw + ss * dw;
              if (wi < 0 || wi >= w) continue;
              const float* xp = x + (((size_t)ni * h + hi) * w + wi) * c + (size_t)g * cg;
              const float* wp = wt + (((((size_t)kk * by + byi) * bx + bxi) * r + rr) * s + ss) * cg;
              for (int32_t ci = 0; ci < cg; ++ci) acc += xp[ci] * wp[ci];
            }
          }
          if (bias) acc += bias[block_bias_index(kk, byi, bxi, by, bx, bias_mode)];
          y[(((size_t)ni * ho_n + ho) * wo_n + wo) * k + kk] = acc;
        }
      }
    }
  }
  return 0;
}

/* cpu_block_bprop_nhwc (cpu_ref.cpp:272-314): as cpu_bprop_nhwc, each tap's output position
 * (ho, wo) taking the filter of its block. */
int orc_block_bprop_f32(const float* dy, int32_t n, int32_t h, int32_t w, int32_t c, const float* wt, int32_t r,
                        int32_t s, int32_t k, const int32_t conv[7], int32_t by, int32_t bx, float* dx,
                        int32_t nthreads) {
  int32_t ho_n, wo_n, bho, bwo;
  if (block_shape(n, h, w, c, r, s, k, conv, by, bx, &ho_n, &wo_n, &bho, &bwo) != 0) return -1;
  const int32_t ph = conv[0], pw = conv[1], sh = conv[2], sw = conv[3], dh = conv[4], dw = conv[5], g_n = conv[6];
  const int32_t cg = c / g_n, kg = k / g_n;
  const int64_t nrows = (int64_t)n * h;
#ifdef _OPENMP
  const int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#else
  (void)nthreads;
#endif
  for (int64_t row = 0; row < nrows; ++row) {
    const int32_t ni = (int32_t)(row / h);
    const int32_t hi = (int32_t)(row % h);
    for (int32_t wi = 0; wi < w; ++wi) {
      for (int32_t g = 0; g < g_n; ++g) {
        for (int32_t ci = 0; ci < cg; ++ci) {
          float acc = 0.0f;
          for (int32_t rr = 0; rr < r; ++rr) {
            const int32_t hn = hi + ph - rr * dh;
            if (hn < 0 || hn % sh != 0) continue;
            const int32_t ho = hn / sh;
            if (ho >= ho_n) continue;
            const int32_t byi = ho / bho;
            for (int32_t ss = 0; ss < s; ++ss) {
              const int32_t wn = wi + pw - ss * dw;
              if (wn < 0 || wn % sw != 0) continue;
              const int32_t wo = wn / sw;
              if (wo >= wo_n) continue;
              const int32_t bxi = wo / bwo;
              for (int32_t ko = 0; ko < kg; ++ko) {
                const int32_t kk = g * kg + ko;
                const float dyv = dy[(((size_t)ni * ho_n + ho) * wo_n + wo) * k + kk];
                const float wv = wt[(((((size_t)kk * by + byi) * bx + bxi) * r + rr) * s + ss) * cg + ci];
                acc += dyv * wv;
              }
            }
          }
          dx[(((size_t)ni * h + hi) * w + wi) * c + (size_t)g * cg + ci] = acc;
        }
      }
    }
  }
  return 0;
}

/* cpu_block_grad_nhwc (cpu_ref.cpp:316-369): dw[k][by][bx][r][s][ci] = sum over n and the
 * block's output positions (in that order, in-bounds taps) of x * dy.  With dbias, every
 * element is first zeroed and dbias[block_bias_index(k, by, bx)] accumulates dy over n and
 * the block's positions, in the reference's loop order (blocks by, bx outermost), counting
 * only positions whose (r, s) = (0, 0) tap lies inside the image (the reference adds dy inside
 * that tap's bounds checks). */
int orc_block_grad_f32(const float* x, int32_t n, int32_t h, int32_t w, int32_t c, const float* dy, int32_t r,
                       int32_t s, int32_t k, const int32_t conv[7], int32_t by, int32_t bx, float* dwt, float* dbias,
                       int32_t bias_mode, int32_t nthreads) {
  int32_t ho_n, wo_n, bho, bwo;
  if (block_shape(n, h, w, c, r, s, k, conv, by, bx, &ho_n, &wo_n, &bho, &bwo) != 0) return -1;
  const int32_t ph = conv[0], pw = conv[1], sh = conv[2], sw = conv[3], dh = conv[4], dw = conv[5], g_n = conv[6];
  const int32_t cg = c / g_n, kg = k / g_n;
  const int64_t nel = (int64_t)k * by * bx * r * s * cg;
#ifdef _OPENMP
  const int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 16) num_threads(nt)
#else
  (void)nthreads;
#endif
  for (int64_t e = 0; e < nel; ++e) {
    const int32_t ci = (int32_t)(e % cg);
    const int32_t ss = (int32_t)((e / cg) % s);
    const int32_t rr = (int32_t)((e / ((int64_t)cg * s)) % r);
    const int32_t bxi = (int32_t)((e / ((int64_t)cg * s * r)) % bx);
    const int32_t byi = (int32_t)((e / ((int64_t)cg * s * r * bx)) % by);
    const int32_t kk = (int32_t)(e / ((int64_t)cg * s * r * bx * by));
    const int32_t g = kk / kg;
    float acc = 0.0f;
    for (int32_t ni = 0; ni < n; ++ni) {
      for (int32_t lho = 0; lho < bho; ++lho) {
        const int32_t ho = byi * bho + lho;
        const int32_t hi = ho * sh - ph + rr * dh;
        if (hi < 0 || hi >= h) continue;
        for (int32_t lwo = 0; lwo < bwo; ++lwo) {
          const int32_t wo = bxi * bwo + lwo;
          const int32_t wi = wo * sw - pw + ss * dw;
          if (wi < 0 || wi >= w) continue;
          acc += x[(((size_t)ni * h + hi) * w + wi) * c + (size_t)g * cg + ci] *
                 dy[(((size_t)ni * ho_n + ho) * wo_n + wo) * k + kk];
        }
      }
    }
    dwt[e] = acc;
  }
  if (dbias) {
    const int64_t nb = (int64_t)k * by * bx;
    for (int64_t i = 0; i < nb; ++i) dbias[i] = 0.0f;
    for (int32_t kk = 0; kk < k; ++kk) {
      for (int32_t byi = 0; byi < by; ++byi) {
        for (int32_t bxi = 0; bxi < bx; ++bxi) {
          float* slot = dbias + block_bias_index(kk, byi, bxi, by, bx, bias_mode);
          for (int32_t ni = 0; ni < n; ++ni) {
            for (int32_t lho = 0; lho < bho; ++lho) {
              const int32_t ho = byi * bho + lho;
              const int32_t hi = ho * sh - ph;
              if (hi < 0 || hi >= h) continue;
              for (int32_t lwo = 0; lwo < bwo; ++lwo) {
                const int32_t wo = bxi * bwo + lwo;
                const int32_t wi = wo * sw - pw;
                if (wi < 0 || wi >= w) continue;
                *slot += dy[(((size_t)ni * ho_n + ho) * wo_n + wo) * k + kk];
              }
            }
          }
        }
      }
    }
  }
  return 0;
}

/* The bias gradient as launch_block_grad_nhwc computes it (cuda_kernels.cu:461-485 and
 * :1112-1119): dy summed over every output position of a block, which the reference adds with
 * float atomics in no fixed order.  Restated here in the fixed order of this library's kernels:
 * a block's positions, in (n, lho, lwo) order, are cut into runs of `chunk` (chunk <= 0: one
 * run), each run is summed from 0, and a slot then adds its runs in order from 0 - mode 0: slot
 * [k][by][bx], its own block's runs; mode 1: slot [k][0][0], every block's runs in (by, bx)
 * order, the other slots 0.  Returns 0, or -1 on a block grid that does not divide ho x wo. */
int orc_block_dbias_f32(const float* dy, int32_t n, int32_t ho_n, int32_t wo_n, int32_t k, int32_t by, int32_t bx,
                        int32_t mode, int32_t chunk, float* dbias) {
  if (by <= 0 || bx <= 0 || ho_n % by != 0 || wo_n % bx != 0) return -1;
  const int32_t bho = ho_n / by, bwo = wo_n / bx;
  const int64_t P = (int64_t)n * bho * bwo;
  const int64_t run = chunk > 0 ? chunk : (P > 0 ? P : 1);
  for (int64_t i = 0; i < (int64_t)k * by * bx; ++i) dbias[i] = 0.0f;
  for (int32_t kk = 0; kk < k; ++kk) {
    for (int32_t byi = 0; byi < by; ++byi) {
      for (int32_t bxi = 0; bxi < bx; ++bxi) {
        float* slot = dbias + block_bias_index(kk, byi, bxi, by, bx, mode);
        for (int64_t p0 = 0; p0 < P; p0 += run) {
          const int64_t p1 = p0 + run < P ? p0 + run : P;
          float part = 0.0f;
          for (int64_t p = p0; p < p1; ++p) {
            const int64_t ni = p / ((int64_t)bho * bwo);
            const int32_t lho = (int32_t)((p / bwo) % bho), lwo = (int32_t)(p % bwo);
            part += dy[(((size_t)ni * ho_n + byi * bho + lho) * wo_n + bxi * bwo + lwo) * k + kk];
          }
          *slot += part;
        }
      }
    }
  }
  return 0;
}
