/*
 * lq_oracle.c -- TEST INFRASTRUCTURE ONLY.  A plain-C CPU restatement of Lucid's
 * quantized-inference arithmetic, used as the parity checker for the HIP backend
 * and (the lqo_lucid_* multi-pass functions) as the timed CPU baseline.  Nothing
 * in lucid_amd/ may link, import or call this file.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp; no -ffast-math, so every
 * float operation is one IEEE binary32 operation in round-to-nearest-even).
 *
 * Citations are into lucid-official/lucid:
 *   F  = lucid/quantization/_functional.py
 *   QP = lucid/quantization/_qparams.py
 *   OB = lucid/quantization/observer.py
 *   BK = lucid/_C/backend/cpu/
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { O_I8 = 1, O_U8 = 2, O_I16 = 3, O_I32 = 4, O_F16 = 5, O_F32 = 6, O_U8S8 = 7 };
enum { O_OBS_MINMAX = 0, O_OBS_EMA = 1, O_OBS_REPLACE = 2 };
enum { O_OUT_I32 = 0, O_OUT_F32 = 1, O_OUT_F16 = 2, O_OUT_Q8 = 3, O_OUT_QU8 = 4,
       O_OUT_FQ32 = 5, O_OUT_Q16 = 6, O_OUT_QU8S8 = 7 };

/* ---------------------------------------------------------------- scalar rules */

/* round half to even: vvnintf (BK/methods/Unary.cpp:143-147, Vforce.h:727-745).
 * nearbyintf in the default FE_TONEAREST mode is exactly that. */
float lqo_rne(float x) { return nearbyintf(x); }

/* clip with NaN pass-through and the signed-zero tie rule of BK/Vdsp.cpp:33-62:
 * a +0 floor also takes -0 (<=), a -0 cap also takes +0 (>=). */
float lqo_clip(float v, float lo, float hi) {
    int lo_ties = (lo == 0.0f) && !signbit(lo);
    int hi_ties = (hi == 0.0f) && signbit(hi);
    if (lo_ties ? v <= lo : v < lo) return lo;
    if (hi_ties ? v >= hi : v > hi) return hi;
    return v;
}

/* extreme of two floats, NaN-propagating, -0 below +0 (BK/Reduce.cpp:54-72). */
float lqo_extreme(float a, float b, int is_max) {
    if (isnan(a) || isnan(b)) return NAN;
    if (is_max) return a > b ? a : (b > a ? b : (signbit(a) ? b : a));
    return a < b ? a : (b < a ? b : (signbit(a) ? a : b));
}

/* float -> integer storage cast: saturating, NaN -> 0 (BK/methods/Factory.cpp:127-146). */
static int64_t satcast(float v, int64_t lo, int64_t hi) {
    if (v != v) return 0;
    if (v <= (float)lo) return lo;
    if (v >= (float)hi) return hi;
    return (int64_t)v; /* truncation toward zero, as static_cast */
}

static void store_code(void* q, int q_dtype, int64_t i, float c) {
    switch (q_dtype) {
    case O_I8: ((int8_t*)q)[i] = (int8_t)satcast(c, -128, 127); break;
    case O_U8: ((uint8_t*)q)[i] = (uint8_t)satcast(c, 0, 255); break;
    case O_I16: ((int16_t*)q)[i] = (int16_t)satcast(c, -32768, 32767); break;
    case O_I32: ((int32_t*)q)[i] = (int32_t)satcast(c, INT32_MIN, INT32_MAX); break;
    case O_U8S8: ((int8_t*)q)[i] = (int8_t)(satcast(c, 0, 255) - 128); break;
    default: break;
    }
}

static float load_code(const void* q, int q_dtype, int64_t i) {
    switch (q_dtype) {
    case O_I8: return (float)((const int8_t*)q)[i];
    case O_U8: return (float)((const uint8_t*)q)[i];
    case O_I16: return (float)((const int16_t*)q)[i];
    case O_I32: return (float)((const int32_t*)q)[i];
    case O_U8S8: return (float)(((const int8_t*)q)[i] + 128);
    default: return 0.0f;
    }
}

/* float32 -> IEEE half, round to nearest even (the conversion numpy's astype(float16)
 * and v_cvt_f16_f32 perform).  Written from the binary16 definition. */
uint16_t lqo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf or nan */
        if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {                                    /* result subnormal or zero */
        /* value = ax as float; half subnormal unit is 2^-24 */
        float a;
        memcpy(&a, &ax, 4);
        float scaled = a * 16777216.0f; /* exact: multiply by 2^24 */
        float r = nearbyintf(scaled);   /* ties to even */
        return (uint16_t)(sign | (uint32_t)r);
    }
    uint32_t exp = (ax >> 23) - 127 + 15;
    uint32_t mant = ax & 0x7fffffu;
    uint32_t h = (exp << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1; /* carry may bump exponent */
    return (uint16_t)(sign | h);
}

float lqo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t x;
    if (exp == 0) {
        float v = (float)mant * (1.0f / 16777216.0f);
        memcpy(&x, &v, 4);
        x |= sign;
    } else if (exp == 31) {
        x = sign | 0x7f800000u | (mant << 13);
    } else {
        x = sign | ((exp - 15 + 127) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* The reciprocal a tensor scale gets: 1.0 / s in float32 (__rtruediv__, _dunders.py:436-466). */
float lqo_recip_f32(float s) { return 1.0f / s; }
/* The reciprocal a Python-float scale gets: 1.0 / s in double, then rounded to float32
 * when the scalar meets the float32 tensor (F:69, _dispatch.py:154-171,308-330). */
float lqo_recip_f64(double s) { return (float)(1.0 / s); }

/* ------------------------------------------------------------- observers */

/* x.min() / x.max() of n floats (BK/Reduce.cpp:74-105): NaN if any NaN, -0 < +0. */
void lqo_minmax_batch(const float* x, int64_t n, float* mn, float* mx) {
    float a = INFINITY, b = -INFINITY;
    for (int64_t i = 0; i < n; ++i) {
        a = lqo_extreme(a, x[i], 0);
        b = lqo_extreme(b, x[i], 1);
    }
    *mn = a;
    *mx = b;
}

/* Fold batch extrema into a running pair (OB:408-414 MinMax; OB:527-544 EMA with
 * new = where(isinf(min_val), cur, m + c*(cur - m))). */
static void fold(float* rmin, float* rmax, float cmin, float cmax, int mode, float c, int first) {
    if (mode == O_OBS_REPLACE) {
        *rmin = cmin;
        *rmax = cmax;
    } else if (mode == O_OBS_MINMAX) {
        *rmin = lqo_extreme(*rmin, cmin, 0); /* lucid.minimum, vDSP_vmin (Vdsp.cpp:196) */
        *rmax = lqo_extreme(*rmax, cmax, 1);
    } else {
        if (first) {
            *rmin = cmin;
            *rmax = cmax;
        } else {
            float dmin = cmin - *rmin;
            float dmax = cmax - *rmax;
            float tmin = c * dmin;
            float tmax = c * dmax;
            *rmin = *rmin + tmin;
            *rmax = *rmax + tmax;
        }
    }
}

void lqo_minmax(const float* x, int64_t n, float* running, int mode, float c) {
    float cmin, cmax;
    lqo_minmax_batch(x, n, &cmin, &cmax);
    fold(&running[0], &running[1], cmin, cmax, mode, c, isinf(running[0]));
}

/* Per-channel (OB:672-685 / OB:1031-1048): x as [outer, C, inner]. */
void lqo_minmax_per_channel(const float* x, int64_t outer, int64_t C, int64_t inner,
                            float* rmin, float* rmax, int mode, float c) {
    int all_inf = 1;
    for (int64_t ch = 0; ch < C; ++ch)
        if (!isinf(rmin[ch])) all_inf = 0;
    for (int64_t ch = 0; ch < C; ++ch) {
        float a = INFINITY, b = -INFINITY;
        for (int64_t o = 0; o < outer; ++o) {
            const float* row = x + (o * C + ch) * inner;
            for (int64_t i = 0; i < inner; ++i) {
                a = lqo_extreme(a, row[i], 0);
                b = lqo_extreme(b, row[i], 1);
            }
        }
        fold(&rmin[ch], &rmax[ch], a, b, mode, c, all_inf);
    }
}

/* calculate_qparams (QP:186-205), elementwise over n ranges. */
void lqo_calc_qparams(const float* mn_in, const float* mx_in, int64_t n, int symmetric,
                      int is_signed, int qmin, int qmax, float eps, float* scale,
                      float* zero_point) {
    for (int64_t i = 0; i < n; ++i) {
        float mn = lqo_extreme(mn_in[i], 0.0f, 0);
        float mx = lqo_extreme(mx_in[i], 0.0f, 1);
        float e = eps;
        if (symmetric) {
            float ma = lqo_extreme(fabsf(mn), fabsf(mx), 1);
            float half = (float)((double)(qmax - qmin) / 2.0);
            float s = lqo_extreme(ma / half, e, 1);
            scale[i] = s;
            zero_point[i] = is_signed ? 0.0f : (float)((qmax + qmin + 1) / 2);
        } else {
            float width = mx - mn;
            float s = lqo_extreme(width / (float)(qmax - qmin), e, 1);
            float r = lqo_rne(mn / s);
            float z = (float)qmin - r;
            scale[i] = s;
            zero_point[i] = lqo_clip(z, (float)qmin, (float)qmax);
        }
    }
}

/* --------------------------------------------------- quantize / dequantize */

/* quantize (F:59-69,190-197) over [outer, C, inner]: inv[c] / zp[c] are per channel
 * (C == 1 with outer*inner == n is the per-tensor case). */
void lqo_quantize(const float* x, int64_t outer, int64_t C, int64_t inner, const float* inv,
                  const float* zp, int qmin, int qmax, void* q, int q_dtype) {
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t ch = 0; ch < C; ++ch)
            for (int64_t i = 0; i < inner; ++i) {
                int64_t idx = (o * C + ch) * inner + i;
                float t = x[idx] * inv[ch];
                float r = lqo_rne(t);
                float u = r + zp[ch];
                float cl = lqo_clip(u, (float)qmin, (float)qmax);
                store_code(q, q_dtype, idx, cl);
            }
}

/* dequantize (F:293): (float(q) - z) * s; y_dtype O_F32 or O_F16. */
void lqo_dequantize(const void* q, int q_dtype, int64_t outer, int64_t C, int64_t inner,
                    const float* s, const float* zp, void* y, int y_dtype) {
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t ch = 0; ch < C; ++ch)
            for (int64_t i = 0; i < inner; ++i) {
                int64_t idx = (o * C + ch) * inner + i;
                float f = load_code(q, q_dtype, idx);
                float d = f - zp[ch];
                float v = d * s[ch];
                if (y_dtype == O_F16)
                    ((uint16_t*)y)[idx] = lqo_f32_to_f16(v);
                else
                    ((float*)y)[idx] = v;
            }
}

/* fake-quantize forward + STE mask (F:314-333). */
void lqo_fake_quantize(const float* x, int64_t outer, int64_t C, int64_t inner,
                       const float* inv, const float* s, const float* zp, int qmin, int qmax,
                       float* y, float* mask) {
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t ch = 0; ch < C; ++ch)
            for (int64_t i = 0; i < inner; ++i) {
                int64_t idx = (o * C + ch) * inner + i;
                float t = x[idx] * inv[ch];
                float r = lqo_rne(t);
                float qpre = r + zp[ch];
                float qc = lqo_clip(qpre, (float)qmin, (float)qmax);
                float d = qc - zp[ch];
                y[idx] = d * s[ch];
                if (mask) {
                    float lo = (qpre >= (float)qmin) ? 1.0f : 0.0f;
                    float hi = (qpre <= (float)qmax) ? 1.0f : 0.0f;
                    mask[idx] = lo * hi;
                }
            }
}

/* ------------------------------------------------------------ W8A8 GEMM */

/* Exact int32 accumulator acc[m,n] = sum_k (A[m,k]-za)(B[n,k]-zb[n]) computed in int64;
 * returns 1 if any accumulator leaves the int32 range (the GEMM contract is then void). */
int lqo_gemm_acc(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb, int64_t M,
                 int64_t N, int64_t K, int32_t za, const int32_t* zb, int32_t* acc) {
    int overflow = 0;
#pragma omp parallel for reduction(| : overflow) schedule(static)
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            int64_t s = 0;
            int32_t z = zb ? zb[n] : 0;
            const int8_t* a = A + m * lda;
            const int8_t* b = B + n * ldb;
            for (int64_t k = 0; k < K; ++k) s += (int64_t)(a[k] - za) * (int64_t)(b[k] - z);
            if (s > INT32_MAX || s < INT32_MIN) overflow = 1;
            acc[m * N + n] = (int32_t)s;
        }
    return overflow;
}

/* Epilogue of the W8A8 contract (one element). */
static void gemm_epilogue_one(int32_t acc, float sa, float sb, const float* bias, int64_t n,
                              float out_inv, float out_s, float out_z, int qmin, int qmax,
                              int out_kind, int relu, void* C, int64_t idx) {
    if (out_kind == O_OUT_I32) {
        ((int32_t*)C)[idx] = acc;
        return;
    }
    float s = sa * sb;
    float y = (float)acc * s;
    if (bias) y = y + bias[n];
    if (relu) y = (y <= 0.0f) ? 0.0f : y; /* BK/Vdsp.cpp vrelu_f32 */
    switch (out_kind) {
    case O_OUT_F32: ((float*)C)[idx] = y; break;
    case O_OUT_F16: ((uint16_t*)C)[idx] = lqo_f32_to_f16(y); break;
    default: {
        float t = y * out_inv;
        float r = lqo_rne(t);
        float u = r + out_z;
        float c = lqo_clip(u, (float)qmin, (float)qmax);
        if (out_kind == O_OUT_Q8) ((int8_t*)C)[idx] = (int8_t)satcast(c, -128, 127);
        else if (out_kind == O_OUT_QU8) ((uint8_t*)C)[idx] = (uint8_t)satcast(c, 0, 255);
        else if (out_kind == O_OUT_Q16) ((int16_t*)C)[idx] = (int16_t)satcast(c, -32768, 32767);
        else if (out_kind == O_OUT_QU8S8) ((int8_t*)C)[idx] = (int8_t)(satcast(c, 0, 255) - 128);
        else { /* FQ32 */
            float d = c - out_z;
            ((float*)C)[idx] = d * out_s;
        }
    }
    }
}

/* Full W8A8 GEMM (C row-major with ldc).  a_scale_stride / b_scale_stride are 0 for
 * a per-tensor scale and 1 for per-row / per-column scales. */
int lqo_gemm_w8a8(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb, void* C,
                  int64_t ldc, int64_t M, int64_t N, int64_t K, const float* a_scale,
                  int64_t a_stride, const float* b_scale, int64_t b_stride, float za_f,
                  const float* zb_f, const float* bias, float out_scale, float out_zp,
                  int qmin, int qmax, int out_kind, int relu) {
    int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * (size_t)(M * N));
    int32_t* zb = NULL;
    if (zb_f) {
        zb = (int32_t*)malloc(sizeof(int32_t) * (size_t)N);
        for (int64_t n = 0; n < N; ++n) zb[n] = (int32_t)zb_f[n];
    }
    int ovf = lqo_gemm_acc(A, lda, B, ldb, M, N, K, (int32_t)za_f, zb, acc);
    float out_inv = 1.0f / out_scale;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n)
            gemm_epilogue_one(acc[m * N + n], a_scale[m * a_stride], b_scale[n * b_stride], bias,
                              n, out_inv, out_scale, out_zp, qmin, qmax, out_kind, relu, C,
                              m * ldc + n);
    free(acc);
    free(zb);
    return ovf;
}

/* Epilogue of the W8A8 contract over a precomputed (already zero-point corrected) int32
 * accumulator acc[M,N]: the same per-element steps as lqo_gemm_w8a8. */
void lqo_gemm_epilogue(const int32_t* acc, int64_t M, int64_t N, const float* a_scale,
                       int64_t a_stride, const float* b_scale, int64_t b_stride,
                       const float* bias, float out_scale, float out_zp, int qmin, int qmax,
                       int out_kind, int relu, void* C, int64_t ldc) {
    float out_inv = 1.0f / out_scale;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n)
            gemm_epilogue_one(acc[m * N + n], a_scale[m * a_stride], b_scale[n * b_stride], bias,
                              n, out_inv, out_scale, out_zp, qmin, qmax, out_kind, relu, C,
                              m * ldc + n);
}

/* ------------------------------------------------- weight-only GEMV (fp64 sum) */

/* y[m,n] = sum_k x[m,k] * w_hat[n,k] + bias[n], w_hat = fl32(fl32(W - zb) * sb), summed
 * in double and rounded once (a tolerance reference: Accelerate's sgemm order is not
 * knowable, BK/methods/Matmul.cpp:80-122). */
void lqo_gemv_w8(const float* x, int64_t M, int64_t K, const int8_t* W, int64_t N,
                 const float* sb, const float* zb, const float* bias, int relu, double* y) {
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t m = 0; m < M; ++m) {
            double s = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                float d = (float)W[n * K + k] - (zb ? zb[n] : 0.0f);
                float w = d * sb[n];
                s += (double)x[m * K + k] * (double)w;
            }
            if (bias) s += (double)bias[n];
            if (relu && s <= 0.0) s = 0.0;
            y[m * N + n] = s;
        }
    }
}

/* ------------------------------------------------------------ convolution */

/* Source index of padded coordinate i for a padding mode (0 zeros, 1 reflect, 2 replicate,
 * 3 circular; torch / Lucid pad semantics, lucid/nn/functional/conv.py:24-29,76-81), or -1
 * for a zero-padded tap. */
static int64_t lqo_pad_index(int64_t i, int64_t n, int mode) {
    if (i >= 0 && i < n) return i;
    if (mode == 1) {
        if (n == 1) return 0;
        int64_t j = i < 0 ? -i : i;
        int64_t period = 2 * (n - 1);
        j %= period;
        return j < n ? j : period - j;
    }
    if (mode == 2) return i < 0 ? 0 : n - 1;
    if (mode == 3) return ((i % n) + n) % n;
    return -1;
}

/* Exact integer convolution of activation codes (stored int8; unsigned-grid codes held as
 * c - 128 when x_u8s8) against weight codes, brute force in int64:
 *   acc[n][co][oh][ow] = sum_{c, kh, kw} (code(x[n][g*Cg+c][h][w]) - za) * w[co][c][kh][kw]
 * with (h, w) the padding-mode image of (oh*sh + kh*dh - pt, ow*sw + kw*dw - pl); a zero-padded
 * tap contributes 0 (its value is the zero point).  Returns 1 if a sum leaves int32. */
int lqo_conv2d_acc(const int8_t* x, int x_u8s8, int za, int64_t N, int64_t C, int64_t H, int64_t W,
                   const int8_t* w, int64_t Cout, int64_t KH, int64_t KW, int sh, int sw, int pt, int pb,
                   int pl, int pr, int dh, int dw, int64_t groups, int mode, int32_t* acc) {
    int64_t OH = (H + pt + pb - (int64_t)dh * (KH - 1) - 1) / sh + 1;
    int64_t OW = (W + pl + pr - (int64_t)dw * (KW - 1) - 1) / sw + 1;
    int64_t Cg = C / groups, Cog = Cout / groups;
    int ovf = 0;
    /* independent outputs; each sum is an exact int64, so the thread split changes nothing */
#pragma omp parallel for collapse(2) reduction(| : ovf) schedule(static)
    for (int64_t n = 0; n < N; ++n)
        for (int64_t co = 0; co < Cout; ++co) {
            int64_t g = co / Cog;
            for (int64_t oh = 0; oh < OH; ++oh)
                for (int64_t ow = 0; ow < OW; ++ow) {
                    int64_t s = 0;
                    for (int64_t c = 0; c < Cg; ++c)
                        for (int64_t kh = 0; kh < KH; ++kh) {
                            int64_t h = lqo_pad_index(oh * sh + kh * dh - pt, H, mode);
                            if (h < 0) continue;
                            for (int64_t kw = 0; kw < KW; ++kw) {
                                int64_t ww = lqo_pad_index(ow * sw + kw * dw - pl, W, mode);
                                if (ww < 0) continue;
                                int64_t code = x[((n * C + g * Cg + c) * H + h) * W + ww];
                                if (x_u8s8) code += 128;
                                s += (code - za) * (int64_t)w[((co * Cg + c) * KH + kh) * KW + kw];
                            }
                        }
                    if (s > INT32_MAX || s < INT32_MIN) ovf = 1;
                    acc[((n * Cout + co) * OH + oh) * OW + ow] = (int32_t)s;
                }
        }
    return ovf;
}

/* Float convolution in the GPU kernel's op order: per output, sum over (c, kh, kw) in that
 * order of fl32(x * w) added in float32 (no FMA), then + bias. */
void lqo_conv2d_f32(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, const float* w,
                    const float* bias, int64_t Cout, int64_t KH, int64_t KW, int sh, int sw, int pt,
                    int pb, int pl, int pr, int dh, int dw, int64_t groups, int mode, float* y) {
    int64_t OH = (H + pt + pb - (int64_t)dh * (KH - 1) - 1) / sh + 1;
    int64_t OW = (W + pl + pr - (int64_t)dw * (KW - 1) - 1) / sw + 1;
    int64_t Cg = C / groups, Cog = Cout / groups;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t co = 0; co < Cout; ++co) {
            int64_t g = co / Cog;
            for (int64_t oh = 0; oh < OH; ++oh)
                for (int64_t ow = 0; ow < OW; ++ow) {
                    float a = 0.0f;
                    for (int64_t c = 0; c < Cg; ++c)
                        for (int64_t kh = 0; kh < KH; ++kh) {
                            int64_t h = lqo_pad_index(oh * sh + kh * dh - pt, H, mode);
                            if (h < 0) continue;
                            for (int64_t kw = 0; kw < KW; ++kw) {
                                int64_t ww = lqo_pad_index(ow * sw + kw * dw - pl, W, mode);
                                if (ww < 0) continue;
                                float prod = x[((n * C + g * Cg + c) * H + h) * W + ww] *
                                             w[((co * Cg + c) * KH + kh) * KW + kw];
                                a = a + prod;
                            }
                        }
                    if (bias) a = a + bias[co];
                    y[((n * Cout + co) * OH + oh) * OW + ow] = a;
                }
        }
}

/* ------------------------------------------- group-wise (MLX-layout) weights */

/* Group-wise affine quantize (formula _qgemm.py:84-97).  A group with max == min gets
 * s_g = 0 and all codes 0, so w_hat = b_g reproduces the constant exactly. */
void lqo_group_quantize(const float* w, int64_t N, int64_t K, int gs, int bits,
                        uint32_t* packed, float* scales, float* biases) {
    int64_t G = K / gs;
    int per_word = 32 / bits;
    uint32_t L = (1u << bits) - 1u;
    int64_t words = K / per_word;
    memset(packed, 0, sizeof(uint32_t) * (size_t)(N * words));
    for (int64_t n = 0; n < N; ++n)
        for (int64_t g = 0; g < G; ++g) {
            const float* p = w + n * K + g * gs;
            float mn = INFINITY, mx = -INFINITY;
            for (int i = 0; i < gs; ++i) {
                mn = lqo_extreme(mn, p[i], 0);
                mx = lqo_extreme(mx, p[i], 1);
            }
            float s = (mx - mn) / (float)L;
            scales[n * G + g] = s;
            biases[n * G + g] = mn;
            for (int i = 0; i < gs; ++i) {
                uint32_t c = 0;
                if (s > 0.0f) {
                    float d = p[i] - mn;
                    float t = d / s;
                    float r = lqo_rne(t);
                    float cl = lqo_clip(r, 0.0f, (float)L);
                    c = (uint32_t)satcast(cl, 0, (int64_t)L);
                }
                int64_t k = g * gs + i;
                packed[n * words + k / per_word] |= c << ((k % per_word) * bits);
            }
        }
}

void lqo_group_dequantize(const uint32_t* packed, const float* scales, const float* biases,
                          int64_t N, int64_t K, int gs, int bits, float* w) {
    int64_t G = K / gs;
    int per_word = 32 / bits;
    uint32_t L = (1u << bits) - 1u;
    int64_t words = K / per_word;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            uint32_t c = (packed[n * words + k / per_word] >> ((k % per_word) * bits)) & L;
            float t = (float)c * scales[n * G + k / gs];
            w[n * K + k] = biases ? t + biases[n * G + k / gs] : t;
        }
}

/* ---------------------------------------- Lucid's literal multi-pass CPU path */
/* These restate how Lucid's CPU backend executes the sidecar ops: one separate
 * full pass per elementwise op, each with its own float32 temporary (Accelerate
 * vDSP/vForce calls, F:69,195-197,293), parallelised over threads for the baseline. */

void lqo_lucid_minmax(const float* x, int64_t n, float* mn, float* mx) {
    float a = INFINITY, b = -INFINITY;
#pragma omp parallel
    {
        float la = INFINITY;
#pragma omp for schedule(static) nowait
        for (int64_t i = 0; i < n; ++i) la = lqo_extreme(la, x[i], 0);
#pragma omp critical
        a = lqo_extreme(a, la, 0);
    }
#pragma omp parallel
    {
        float lb = -INFINITY;
#pragma omp for schedule(static) nowait
        for (int64_t i = 0; i < n; ++i) lb = lqo_extreme(lb, x[i], 1);
#pragma omp critical
        b = lqo_extreme(b, lb, 1);
    }
    *mn = a;
    *mx = b;
}

/* quantize: mul, round, add, clip, cast -- five passes, four float32 temporaries. */
void lqo_lucid_quantize(const float* x, int64_t n, float inv, float z, int qmin, int qmax,
                        int8_t* q, float* t0, float* t1) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) t0[i] = x[i] * inv;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) t1[i] = lqo_rne(t0[i]);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) t0[i] = t1[i] + z;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) t1[i] = lqo_clip(t0[i], (float)qmin, (float)qmax);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) q[i] = (int8_t)satcast(t1[i], -128, 127);
}

/* dequantize: cast, sub, mul -- three passes. */
void lqo_lucid_dequantize(const int8_t* q, int64_t n, float s, float z, float* y, float* t0) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) t0[i] = (float)q[i];
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) t0[i] = t0[i] - z;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) y[i] = t0[i] * s;
}

int lqo_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

/* The division by 6 of the GPU hardsigmoid / hardswish (lucid_amd/csrc/lq_act.hip): a
 * multiply by fl32(1/6) corrected by one fma residual step where 2^-125 <= |t| <= FLT_MAX, the
 * IEEE division elsewhere.  Returns how many of the 2^32 float32 inputs t (NaNs skipped) give
 * a result other than the IEEE quotient fl32(t / 6) that Lucid computes
 * (backend/cpu/methods/Activation.cpp:680, 743); the rewrite is valid iff this is 0. */
int64_t lqo_div6_mismatches(void) {
    const float r = 1.0f / 6.0f;
    int64_t bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (int64_t i = 0; i < (int64_t)1 << 32; ++i) {
        const uint32_t u = (uint32_t)i;
        float t;
        memcpy(&t, &u, 4);
        if (t != t) continue;
        const float want = t / 6.0f;
        float q;
        const float a = fabsf(t);
        if (a >= 0x1p-125f && a <= FLT_MAX) {
            const float q0 = t * r;
            const float e = fmaf(-q0, 6.0f, t);
            q = fmaf(e, r, q0);
        } else {
            q = t / 6.0f;
        }
        uint32_t uq, uw;
        memcpy(&uq, &q, 4);
        memcpy(&uw, &want, 4);
        bad += uq != uw;
    }
    return bad;
}
