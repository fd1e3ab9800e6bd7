// lq_pool.hip -- 2-D max and average pooling (fixed windows and adaptive cells) over float32
// or over the integer codes of a code-backed activation.
//
// Lucid's CPU kernels (lucid/_C/backend/cpu/Pool.cpp:27-32, 57-100, 117-168) and its adaptive
// cells (lucid/nn/functional/_pool_core.py:228-250, 407-434):
//   max  first in-window element, then replaced by v when v > best or v is NaN and best is
//        not (NaN propagates); padding positions are skipped
//   avg  float32 sum of the in-window elements in row-major order, then sum / denom, denom
//        the window size with (count_include_pad) or without padding; 0 for an empty window
//   adaptive cell o of S -> O: [floor(o S / O), ceil((o + 1) S / O)), averaged over its size
// Codes: the max of codes is the code of the max (dequantization is increasing for a positive
// scale), so max pooling keeps the input grid and moves bytes only; average pooling
// dequantizes each element (fl32(fl32(c - z) * s)) and outputs float32, as the reference pools
// the fake-quantized floats.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "lq_internal.h"

namespace lq {

struct PoolArgs {
    const void* x;
    int x_type;
    const float* x_scale;
    const float* x_zp;
    int64_t NC;
    int H, W, OH, OW, KH, KW, sh, sw, ph, pw;
    int adaptive, count_include_pad;
    void* y;
};

template <int T>
struct PoolElem;
template <> struct PoolElem<LQ_F32> { using type = float; };
template <> struct PoolElem<LQ_I8> { using type = int8_t; };
template <> struct PoolElem<LQ_U8> { using type = uint8_t; };
template <> struct PoolElem<LQ_I16> { using type = int16_t; };
template <> struct PoolElem<LQ_U8S8> { using type = int8_t; };

__device__ __forceinline__ void pool_window(const PoolArgs& a, int o, int S, int O, int K, int st, int p, int& lo,
                                            int& hi, int& span) {
    if (a.adaptive) {
        lo = (int)(((int64_t)o * S) / O);
        hi = (int)(((int64_t)(o + 1) * S + O - 1) / O);
        span = hi - lo;
        return;
    }
    const int start = o * st - p;
    const int end = min(start + K, S + p);
    lo = max(start, 0);
    hi = min(end, S);
    span = a.count_include_pad ? end - start : (hi > lo ? hi - lo : 0);
}

// (nc, oh, ow) of flat output index i: 32-bit divisions when the output count fits (a 64-bit
// division is a long instruction sequence on this GPU, and three per output dominated the
// pooling kernels).
__device__ __forceinline__ void pool_coords(const PoolArgs& a, int64_t i, int64_t total, int64_t& nc, int& oh,
                                            int& ow) {
    if (total <= 0x7fffffff) {
        const uint32_t u = (uint32_t)i, q = u / (uint32_t)a.OW;
        ow = (int)(u - q * (uint32_t)a.OW);
        const uint32_t r = q / (uint32_t)a.OH;
        oh = (int)(q - r * (uint32_t)a.OH);
        nc = r;
    } else {
        ow = (int)(i % a.OW);
        const int64_t t = i / a.OW;
        oh = (int)(t % a.OH);
        nc = t / a.OH;
    }
}

template <int T>
__global__ __launch_bounds__(256) void max_pool_kernel(PoolArgs a) {
    using E = typename PoolElem<T>::type;
    const int64_t total = a.NC * a.OH * a.OW;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        int64_t nc;
        int oh, ow;
        pool_coords(a, i, total, nc, oh, ow);
        int h0, h1, w0, w1, sp;
        pool_window(a, oh, a.H, a.OH, a.KH, a.sh, a.ph, h0, h1, sp);
        pool_window(a, ow, a.W, a.OW, a.KW, a.sw, a.pw, w0, w1, sp);
        const E* xb = static_cast<const E*>(a.x) + nc * a.H * a.W;
        E best = E(0);
        bool any = false;
        for (int h = h0; h < h1; ++h)
            for (int w = w0; w < w1; ++w) {
                const E v = xb[h * a.W + w];
                bool take = !any || v > best;
                if constexpr (T == LQ_F32) take = take || (v != v && !(best != best));
                if (take) best = v;
                any = true;
            }
        if constexpr (T == LQ_F32) {
            if (!any) best = -__builtin_inff();
        }
        static_cast<E*>(a.y)[i] = best;
    }
}

template <int T>
__device__ __forceinline__ float pool_load(const PoolArgs& a, const typename PoolElem<T>::type* p, float s, float z) {
    if constexpr (T == LQ_F32) {
        return *p;
    } else {
        const float c = (T == LQ_U8S8) ? (float)((int)*p + 128) : (float)*p;
        const float d = c - z;
        return d * s;
    }
}

template <int T>
__global__ __launch_bounds__(256) void avg_pool_kernel(PoolArgs a) {
    using E = typename PoolElem<T>::type;
    const float s = a.x_scale ? a.x_scale[0] : 1.0f, z = a.x_zp ? a.x_zp[0] : 0.0f;
    const int64_t total = a.NC * a.OH * a.OW;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        int64_t nc;
        int oh, ow;
        pool_coords(a, i, total, nc, oh, ow);
        int h0, h1, w0, w1, sph, spw;
        pool_window(a, oh, a.H, a.OH, a.KH, a.sh, a.ph, h0, h1, sph);
        pool_window(a, ow, a.W, a.OW, a.KW, a.sw, a.pw, w0, w1, spw);
        const E* xb = static_cast<const E*>(a.x) + nc * a.H * a.W;
        float sum = 0.0f;
        for (int h = h0; h < h1; ++h)
            for (int w = w0; w < w1; ++w) sum = sum + pool_load<T>(a, xb + h * a.W + w, s, z);
        const int denom = sph * spw;
        static_cast<float*>(a.y)[i] = denom > 0 ? sum / (float)denom : 0.0f;
    }
}

// Plane-staged pooling: a workgroup owns pp consecutive (n, c) planes, which are contiguous in
// memory.  It copies their bytes into LDS with 16-byte loads (byte loads for the partial chunks
// at the tensor's ends, or everywhere when x is not 16-byte aligned), then computes each output
// from LDS with the same window rules and the same element order as the per-output kernels
// above, so the results are identical; only the global traffic changes (one coalesced read of
// each plane instead of one narrow load per window element per output).
constexpr int POOL_PLANE_LDS = 24576;  // bytes of planes per workgroup (two workgroups per CU or more)

template <int T, bool MAX>
__global__ __launch_bounds__(256) void pool_planes_kernel(PoolArgs a, int pp, int64_t total_bytes, int aligned) {
    using E = typename PoolElem<T>::type;
    extern __shared__ __attribute__((aligned(16))) uint8_t pool_lds[];
    const int tid = threadIdx.x;
    const int64_t HW = (int64_t)a.H * a.W;
    const int64_t nc0 = (int64_t)blockIdx.x * pp;
    const int np = (int)min((int64_t)pp, a.NC - nc0);
    const int64_t b0 = nc0 * HW * (int64_t)sizeof(E), b1 = (nc0 + np) * HW * (int64_t)sizeof(E);
    const int64_t c0 = b0 & ~(int64_t)15, c1 = (b1 + 15) & ~(int64_t)15;
    const uint8_t* xb = static_cast<const uint8_t*>(a.x);
    for (int64_t c = c0 + 16 * tid; c < c1; c += 16 * 256) {
        uint8_t* dst = pool_lds + (c - c0);
        if (aligned && c + 16 <= total_bytes) {
            *reinterpret_cast<int4*>(dst) = *reinterpret_cast<const int4*>(xb + c);
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e)
                if (c + e < total_bytes) dst[e] = xb[c + e];
        }
    }
    __syncthreads();
    const E* P = reinterpret_cast<const E*>(pool_lds + (b0 - c0));  // b0 - c0 is a multiple of sizeof(E)
    const int OHW = a.OH * a.OW;
    const float s = a.x_scale ? a.x_scale[0] : 1.0f, z = a.x_zp ? a.x_zp[0] : 0.0f;
    // work item = (plane, output column, row group): the column window is computed once, the
    // rows og, og + G, ... follow (G row groups keep the 256 threads busy on narrow planes)
    const int cols = np * a.OW;
    const int G = max(1, min(a.OH, 256 / max(cols, 1)));
    for (int item = tid; item < cols * G; item += 256) {
        const int og = item / cols, c = item - og * cols;
        const int pl = c / a.OW, ow = c - pl * a.OW;
        int w0, w1, spw;
        pool_window(a, ow, a.W, a.OW, a.KW, a.sw, a.pw, w0, w1, spw);
        const E* xp = P + (int64_t)pl * HW;
        const int64_t o0 = (nc0 + pl) * OHW + ow;
        if constexpr (MAX && T != LQ_F32) {
            // integer codes: the window maximum, order-free, so rows and columns outside the
            // window are clamped onto its edge (a repeated element leaves the maximum alone)
            // and fixed windows up to 3 x 3 run unrolled and branch-free
            if (!a.adaptive && a.KH <= 3 && a.KW <= 3) {
                int wc[3];
#pragma unroll
                for (int k = 0; k < 3; ++k) wc[k] = min(max(ow * a.sw - a.pw + min(k, a.KW - 1), w0), w1 - 1);
                for (int oh = og; oh < a.OH; oh += G) {
                    int h0, h1, sph;
                    pool_window(a, oh, a.H, a.OH, a.KH, a.sh, a.ph, h0, h1, sph);
                    int best = (int)xp[h0 * a.W + w0];
#pragma unroll
                    for (int kh = 0; kh < 3; ++kh) {
                        const int hh = min(max(oh * a.sh - a.ph + min(kh, a.KH - 1), h0), h1 - 1);
                        const E* row = xp + hh * a.W;
#pragma unroll
                        for (int k = 0; k < 3; ++k) best = max(best, (int)row[wc[k]]);
                    }
                    static_cast<E*>(a.y)[o0 + (int64_t)oh * a.OW] = (E)best;
                }
                continue;
            }
        }
        for (int oh = og; oh < a.OH; oh += G) {
            int h0, h1, sph;
            pool_window(a, oh, a.H, a.OH, a.KH, a.sh, a.ph, h0, h1, sph);
            const int64_t o = o0 + (int64_t)oh * a.OW;
            if constexpr (MAX) {
                E best = E(0);
                bool any = false;
                for (int h = h0; h < h1; ++h)
                    for (int w = w0; w < w1; ++w) {
                        const E v = xp[h * a.W + w];
                        bool take = !any || v > best;
                        if constexpr (T == LQ_F32) take = take || (v != v && !(best != best));
                        if (take) best = v;
                        any = true;
                    }
                if constexpr (T == LQ_F32) {
                    if (!any) best = -__builtin_inff();
                }
                static_cast<E*>(a.y)[o] = best;
            } else {
                float sum = 0.0f;
                for (int h = h0; h < h1; ++h)
                    for (int w = w0; w < w1; ++w) sum = sum + pool_load<T>(a, xp + h * a.W + w, s, z);
                const int denom = sph * spw;
                static_cast<float*>(a.y)[o] = denom > 0 ? sum / (float)denom : 0.0f;
            }
        }
    }
}

// ---- into / out of the padded NHWC layout of lq_conv2d_i8_nhwc
//
// Max pooling of byte codes from NCHW planes into that layout, for the first convolution of a
// network whose later layers stay NHWC (the ResNet stem's pool).  A workgroup owns (image n,
// output row oh, 64 channels): it stages the window's input rows of its channels in LDS (16-byte
// loads when rows are aligned), then writes the row's OW pixels x 64 channels, four channels
// per thread, the channels of a pixel contiguous; and its share of the border (the left and
// right border pixels of its row, the top / bottom border rows for the first / last row) with
// the zero point's code.  The window rules are pool_window's and the maximum is order-free,
// so the codes are lq_pool2d's.
constexpr int MPN_MAX_K = 3;
struct MaxNhwcArgs {
    const int8_t* x;
    int C, H, W, OH, OW, KH, KW, sh, sw, ph, pw;
    int8_t* y;
    int ypad, ycs;
    int64_t yrow, yimg;
    const float* zp;
};

template <int T>
__global__ __launch_bounds__(256) void maxpool_to_nhwc_kernel(MaxNhwcArgs a) {
    extern __shared__ __attribute__((aligned(16))) int8_t mp_lds[];  // [64 ch][KH rows][W]
    const int oh = blockIdx.x, n = blockIdx.y, cg = blockIdx.z * 64;
    const int tid = threadIdx.x;
    PoolArgs pa{};
    pa.adaptive = 0;
    int h0, h1, sp;
    pool_window(pa, oh, a.H, a.OH, a.KH, a.sh, a.ph, h0, h1, sp);
    const int nr = h1 - h0;
    const int nch = min(64, a.C - cg);
    const bool vec = (a.W & 15) == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0;
    const int rowq = a.W >> 4;
    if (vec) {
        for (int i = tid; i < nch * nr * rowq; i += 256) {
            const int q = i % rowq, rc = i / rowq, r = rc % nr, c = rc / nr;
            const int8_t* src = a.x + (((int64_t)n * a.C + cg + c) * a.H + h0 + r) * a.W + 16 * q;
            *reinterpret_cast<int4*>(mp_lds + (c * MPN_MAX_K + r) * a.W + 16 * q) = *reinterpret_cast<const int4*>(src);
        }
    } else {
        for (int i = tid; i < nch * nr * a.W; i += 256) {
            const int w = i % a.W, rc = i / a.W, r = rc % nr, c = rc / nr;
            mp_lds[(c * MPN_MAX_K + r) * a.W + w] = a.x[(((int64_t)n * a.C + cg + c) * a.H + h0 + r) * a.W + w];
        }
    }
    __syncthreads();
    const int zi = (int)a.zp[0];
    const uint32_t zc = (uint8_t)(T == LQ_U8S8 ? zi - 128 : zi);
    const uint32_t zc4 = zc * 0x01010101u;
    int8_t* yrow = a.y + (int64_t)n * a.yimg + (int64_t)(oh + a.ypad) * a.yrow;
    for (int i = tid; i < a.OW * (nch >> 2); i += 256) {
        const int ow = i / (nch >> 2), c4 = 4 * (i - ow * (nch >> 2));
        int w0, w1;
        pool_window(pa, ow, a.W, a.OW, a.KW, a.sw, a.pw, w0, w1, sp);
        uint32_t packed = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int8_t* rows = mp_lds + (c4 + e) * MPN_MAX_K * a.W;
            int best = T == LQ_U8 ? (int)(uint8_t)rows[w0] : (int)rows[w0];
            for (int r = 0; r < nr; ++r)
                for (int w = w0; w < w1; ++w) {
                    const int v = T == LQ_U8 ? (int)(uint8_t)rows[r * a.W + w] : (int)rows[r * a.W + w];
                    best = max(best, v);
                }
            packed |= ((uint32_t)best & 0xffu) << (8 * e);
        }
        *reinterpret_cast<uint32_t*>(yrow + (int64_t)(ow + a.ypad) * a.ycs + cg + c4) = packed;
    }
    if (a.ypad) {
        // this row's left and right border pixels, and the top / bottom border rows
        for (int i = tid; i < 2 * (nch >> 2); i += 256) {
            const int side = i / (nch >> 2), c4 = 4 * (i - side * (nch >> 2));
            *reinterpret_cast<uint32_t*>(yrow + (int64_t)(side ? a.OW + a.ypad : 0) * a.ycs + cg + c4) = zc4;
        }
        if (oh == 0 || oh == a.OH - 1) {
            const int wp = a.OW + 2 * a.ypad;
            for (int i = tid; i < wp * (nch >> 2); i += 256) {
                const int px = i / (nch >> 2), c4 = 4 * (i - px * (nch >> 2));
                if (oh == 0) *reinterpret_cast<uint32_t*>(yrow - a.yrow + (int64_t)px * a.ycs + cg + c4) = zc4;
                if (oh == a.OH - 1)
                    *reinterpret_cast<uint32_t*>(yrow + a.yrow + (int64_t)px * a.ycs + cg + c4) = zc4;
            }
        }
    }
}

// Max pooling within the padded NHWC layout (input border x_pad, any content: windows never
// read it): one thread per (pixel, 16 channels), the window's 16-byte vectors compared byte by
// byte; the output border gets the zero point's code.  The same window rules and order-free
// maximum as lq_pool2d.
struct MaxNhwc2Args {
    const int8_t* x;
    int N, C, H, W, xpad, xcs, OH, OW, KH, KW, sh, sw, ph, pw;
    int8_t* y;
    int ypad, ycs;
    const float* zp;
};

template <int T>
__device__ __forceinline__ int byte_val(uint32_t w, int e) {
    const uint32_t b = (w >> (8 * e)) & 0xffu;
    return T == LQ_U8 ? (int)b : (int)(int8_t)(uint8_t)b;
}

template <int T>
__global__ __launch_bounds__(256) void maxpool_nhwc_kernel(MaxNhwc2Args a) {
    const int chunks = a.C >> 4;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = (int64_t)a.N * a.OH * a.OW * chunks;
    if (i >= total) return;
    const int ch = (int)(i % chunks);
    const int64_t pix = i / chunks;
    const int ow = (int)(pix % a.OW);
    const int64_t t = pix / a.OW;
    const int oh = (int)(t % a.OH), n = (int)(t / a.OH);
    PoolArgs pa{};
    int h0, h1, w0, w1, sp;
    pool_window(pa, oh, a.H, a.OH, a.KH, a.sh, a.ph, h0, h1, sp);
    pool_window(pa, ow, a.W, a.OW, a.KW, a.sw, a.pw, w0, w1, sp);
    const int64_t xrow = (int64_t)(a.W + 2 * a.xpad) * a.xcs;
    const int8_t* xb = a.x + ((int64_t)n * (a.H + 2 * a.xpad) + a.xpad) * xrow + (int64_t)a.xpad * a.xcs + 16 * ch;
    vu4 v[MPN_MAX_K * MPN_MAX_K];
    int nv = 0;
#pragma unroll
    for (int kh = 0; kh < MPN_MAX_K; ++kh)
#pragma unroll
        for (int kw = 0; kw < MPN_MAX_K; ++kw) {
            const int h = min(h0 + kh, h1 - 1), w = min(w0 + kw, w1 - 1);  // repeats leave the max alone
            v[kh * MPN_MAX_K + kw] = *reinterpret_cast<const vu4*>(xb + (int64_t)h * xrow + (int64_t)w * a.xcs);
            ++nv;
        }
    uint32_t out[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        uint32_t o = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            int best = byte_val<T>(v[0][d], e);
#pragma unroll
            for (int k = 1; k < MPN_MAX_K * MPN_MAX_K; ++k) best = max(best, byte_val<T>(v[k][d], e));
            o |= ((uint32_t)best & 0xffu) << (8 * e);
        }
        out[d] = o;
    }
    const int64_t yrow = (int64_t)(a.OW + 2 * a.ypad) * a.ycs;
    int8_t* yp = a.y + ((int64_t)n * (a.OH + 2 * a.ypad) + oh + a.ypad) * yrow + (int64_t)(ow + a.ypad) * a.ycs + 16 * ch;
    *reinterpret_cast<vu4*>(yp) = vu4{out[0], out[1], out[2], out[3]};
    if (a.ypad) {
        const int zi = (int)a.zp[0];
        const uint32_t z4 = (uint32_t)(uint8_t)(T == LQ_U8S8 ? zi - 128 : zi) * 0x01010101u;
        const vu4 zc = vu4{z4, z4, z4, z4};
        const bool l = ow == 0, r = ow == a.OW - 1;
        const int64_t cs = a.ycs;
        if (l) *reinterpret_cast<vu4*>(yp - cs) = zc;
        if (r) *reinterpret_cast<vu4*>(yp + cs) = zc;
        if (oh == 0) {
            *reinterpret_cast<vu4*>(yp - yrow) = zc;
            if (l) *reinterpret_cast<vu4*>(yp - yrow - cs) = zc;
            if (r) *reinterpret_cast<vu4*>(yp - yrow + cs) = zc;
        }
        if (oh == a.OH - 1) {
            *reinterpret_cast<vu4*>(yp + yrow) = zc;
            if (l) *reinterpret_cast<vu4*>(yp + yrow - cs) = zc;
            if (r) *reinterpret_cast<vu4*>(yp + yrow + cs) = zc;
        }
    }
}

// y[n][c] = (sum over h, then w, of fl32(fl32(float(code) - z) s)) / (H W): the adaptive
// average pool to 1 x 1 (lq_pool2d's order and rounding) from the padded NHWC layout.  One
// thread per (n, c): consecutive threads read consecutive channel bytes of a pixel.
// One thread per (n, c), 64 per workgroup (N C / 64 workgroups: 256 for ResNet-18 at batch 32,
// one per CU, where 256-thread workgroups left three quarters of the CUs idle).
constexpr int AVG_NHWC_THREADS = 64;
constexpr int AVG_NHWC_BATCH = 64;  // pixel loads in flight per thread (7 x 7 in one round trip)
template <int T>
__global__ __launch_bounds__(AVG_NHWC_THREADS) void avgpool_global_nhwc_kernel(const int8_t* __restrict__ x,
                                                                               int64_t N, int C, int H, int W,
                                                                               int xpad, int xcs, const float* scale,
                                                                               const float* zp,
                                                                               float* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * AVG_NHWC_THREADS + threadIdx.x;
    if (i >= N * C) return;
    const int64_t n = i / C;
    const int c = (int)(i - n * C);
    const float s = scale[0], z = zp ? zp[0] : 0.0f;
    const int64_t wp = W + 2 * xpad;
    const int8_t* base = x + ((n * (H + 2 * xpad) + xpad) * wp + xpad) * xcs + c;
    // the pixels' bytes in batches of AVG_NHWC_BATCH loads, then added in (h, w) order
    float sum = 0.0f;
    const int HW = H * W;
    for (int k0 = 0; k0 < HW; k0 += AVG_NHWC_BATCH) {
        int8_t b[AVG_NHWC_BATCH];
        int h = k0 / W, w = k0 - h * W;  // pixel k0 + u, advanced without a division per load
#pragma unroll
        for (int u = 0; u < AVG_NHWC_BATCH; ++u) {
            b[u] = base[((int64_t)min(h, H - 1) * wp + w) * xcs];
            if (++w == W) w = 0, ++h;
        }
#pragma unroll
        for (int u = 0; u < AVG_NHWC_BATCH; ++u)
            if (k0 + u < HW) {
                const float cv = T == LQ_U8S8 ? (float)((int)b[u] + 128) : T == LQ_U8 ? (float)(uint8_t)b[u] : (float)b[u];
                const float d = cv - z;
                sum = sum + d * s;
            }
    }
    y[i] = sum / (float)HW;
}

}  // namespace lq

using namespace lq;

extern "C" {

int lq_pool2d(int op, const void* d_x, int x_type, const float* d_x_scale, const float* d_x_zero_point, int64_t N,
              int64_t C, int64_t H, int64_t W, int64_t OH, int64_t OW, int KH, int KW, int stride_h, int stride_w,
              int pad_h, int pad_w, int flags, void* d_y, void* stream) {
    LQ_REQUIRE(op == LQ_POOL_MAX || op == LQ_POOL_AVG, "lq_pool2d: op must be LQ_POOL_MAX or LQ_POOL_AVG");
    LQ_REQUIRE(x_type == LQ_F32 || x_type == LQ_I8 || x_type == LQ_U8 || x_type == LQ_I16 || x_type == LQ_U8S8,
               "lq_pool2d: unsupported element type");
    LQ_REQUIRE(N >= 0 && C >= 0 && H >= 1 && W >= 1 && OH >= 0 && OW >= 0 && H < (1 << 30) && W < (1 << 30),
               "lq_pool2d: bad shape");
    LQ_REQUIRE((flags & ~(LQ_POOL_ADAPTIVE | LQ_POOL_COUNT_INCLUDE_PAD)) == 0, "lq_pool2d: unknown flags");
    const bool adaptive = (flags & LQ_POOL_ADAPTIVE) != 0;
    if (!adaptive) {
        LQ_REQUIRE(KH >= 1 && KW >= 1 && stride_h >= 1 && stride_w >= 1 && pad_h >= 0 && pad_w >= 0 &&
                       2 * pad_h <= KH && 2 * pad_w <= KW,
                   "lq_pool2d: kernel / stride / padding out of range (padding at most half the window)");
        LQ_REQUIRE(OH == (H + 2 * pad_h - KH) / stride_h + 1 && OW == (W + 2 * pad_w - KW) / stride_w + 1 &&
                       H + 2 * pad_h >= KH && W + 2 * pad_w >= KW,
                   "lq_pool2d: output size does not match the window");
    } else {
        LQ_REQUIRE(OH >= 1 && OW >= 1, "lq_pool2d: adaptive output size must be positive");
    }
    LQ_REQUIRE(op == LQ_POOL_MAX || x_type == LQ_F32 || d_x_scale, "lq_pool2d: average of codes needs the scale");
    const int64_t total = N * C * OH * OW;
    if (total == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y, "lq_pool2d: NULL pointer");
    PoolArgs a{d_x, x_type, x_type == LQ_F32 ? nullptr : d_x_scale, x_type == LQ_F32 ? nullptr : d_x_zero_point,
               N * C, (int)H, (int)W, (int)OH, (int)OW, KH, KW, stride_h, stride_w, pad_h, pad_w, adaptive ? 1 : 0,
               (flags & LQ_POOL_COUNT_INCLUDE_PAD) ? 1 : 0, d_y};
    hipStream_t st = as_stream(stream);
    const int esz = x_type == LQ_F32 ? 4 : x_type == LQ_I16 ? 2 : 1;
    const int64_t plane_bytes = H * W * esz;
    if (plane_bytes <= POOL_PLANE_LDS && N * C < ((int64_t)1 << 31)) {
        // planes per workgroup: as many as the LDS budget holds, but no fewer than ~1024
        // workgroups when there are that many planes (small planes: a thread per column)
        const int64_t nc = N * C;
        const int pp = (int)std::max<int64_t>(1, std::min<int64_t>(POOL_PLANE_LDS / plane_bytes, (nc + 1023) / 1024));
        const int64_t blocks = (N * C + pp - 1) / pp;
        const size_t lds = (size_t)(((int64_t)pp * plane_bytes + 15) / 16 * 16 + 16);
        const int al = (reinterpret_cast<uintptr_t>(d_x) & 15) == 0 ? 1 : 0;
        const int64_t tb = N * C * plane_bytes;
        const dim3 pg((unsigned)blocks);
#define LQ_POOL_PLANES(MX)                                                                                   \
    switch (x_type) {                                                                                        \
        case LQ_F32: hipLaunchKernelGGL((pool_planes_kernel<LQ_F32, MX>), pg, dim3(256), lds, st, a, pp, tb, al); break; \
        case LQ_I8: hipLaunchKernelGGL((pool_planes_kernel<LQ_I8, MX>), pg, dim3(256), lds, st, a, pp, tb, al); break;   \
        case LQ_U8: hipLaunchKernelGGL((pool_planes_kernel<LQ_U8, MX>), pg, dim3(256), lds, st, a, pp, tb, al); break;   \
        case LQ_I16: hipLaunchKernelGGL((pool_planes_kernel<LQ_I16, MX>), pg, dim3(256), lds, st, a, pp, tb, al); break; \
        default: hipLaunchKernelGGL((pool_planes_kernel<LQ_U8S8, MX>), pg, dim3(256), lds, st, a, pp, tb, al); break;    \
    }
        if (op == LQ_POOL_MAX) {
            LQ_POOL_PLANES(true)
        } else {
            LQ_POOL_PLANES(false)
        }
#undef LQ_POOL_PLANES
        note_path("pool planes");
        return launch_status("lq_pool2d");
    }
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    const dim3 grid((unsigned)blocks);
#define LQ_POOL_LAUNCH(K)                                                                               \
    switch (x_type) {                                                                                   \
        case LQ_F32: hipLaunchKernelGGL(K<LQ_F32>, grid, dim3(256), 0, st, a); break;                   \
        case LQ_I8: hipLaunchKernelGGL(K<LQ_I8>, grid, dim3(256), 0, st, a); break;                     \
        case LQ_U8: hipLaunchKernelGGL(K<LQ_U8>, grid, dim3(256), 0, st, a); break;                     \
        case LQ_I16: hipLaunchKernelGGL(K<LQ_I16>, grid, dim3(256), 0, st, a); break;                   \
        default: hipLaunchKernelGGL(K<LQ_U8S8>, grid, dim3(256), 0, st, a); break;                      \
    }
    if (op == LQ_POOL_MAX) {
        LQ_POOL_LAUNCH(max_pool_kernel)
    } else {
        LQ_POOL_LAUNCH(avg_pool_kernel)
    }
#undef LQ_POOL_LAUNCH
    note_path("pool per output");
    return launch_status("lq_pool2d");
}

int lq_maxpool2d_i8_to_nhwc(const int8_t* d_x, int x_type, const float* d_zero_point, int64_t N, int64_t C,
                            int64_t H, int64_t W, int64_t OH, int64_t OW, int KH, int KW, int stride_h, int stride_w,
                            int pad_h, int pad_w, int8_t* d_y, int y_pad, int64_t y_cs, void* stream) {
    const char* fn = "lq_maxpool2d_i8_to_nhwc";
    LQ_REQUIRE(x_type == LQ_I8 || x_type == LQ_U8 || x_type == LQ_U8S8, std::string(fn) + ": byte codes expected");
    LQ_REQUIRE(N >= 0 && C >= 1 && H >= 1 && W >= 1 && KH >= 1 && KW >= 1 && KH <= MPN_MAX_K && KW <= MPN_MAX_K &&
                   stride_h >= 1 && stride_w >= 1 && pad_h >= 0 && pad_w >= 0 && 2 * pad_h <= KH && 2 * pad_w <= KW,
               std::string(fn) + ": windows up to 3 x 3, padding at most half the window");
    LQ_REQUIRE(OH == (H + 2 * pad_h - KH) / stride_h + 1 && OW == (W + 2 * pad_w - KW) / stride_w + 1 &&
                   H + 2 * pad_h >= KH && W + 2 * pad_w >= KW,
               std::string(fn) + ": output size does not match the window");
    LQ_REQUIRE(C % 16 == 0 && y_cs == C && y_pad >= 0 && y_pad <= 1,
               std::string(fn) + ": C a multiple of 16, y_cs == C, a border of 0 or 1");
    LQ_REQUIRE((int64_t)MPN_MAX_K * W * 64 <= 65536 && OH <= 65535 && N <= 65535, std::string(fn) + ": too large");
    if (N == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y && d_zero_point, std::string(fn) + ": NULL pointer");
    MaxNhwcArgs a{};
    a.x = d_x;
    a.C = (int)C; a.H = (int)H; a.W = (int)W; a.OH = (int)OH; a.OW = (int)OW;
    a.KH = KH; a.KW = KW; a.sh = stride_h; a.sw = stride_w; a.ph = pad_h; a.pw = pad_w;
    a.y = d_y;
    a.ypad = y_pad;
    a.ycs = (int)y_cs;
    a.yrow = (OW + 2 * y_pad) * y_cs;
    a.yimg = (OH + 2 * y_pad) * a.yrow;
    a.zp = d_zero_point;
    const dim3 grid((unsigned)OH, (unsigned)N, (unsigned)((C + 63) / 64));
    const size_t lds = (size_t)MPN_MAX_K * W * 64;
    const hipStream_t st = as_stream(stream);
    if (x_type == LQ_I8) hipLaunchKernelGGL(maxpool_to_nhwc_kernel<LQ_I8>, grid, dim3(256), lds, st, a);
    else if (x_type == LQ_U8) hipLaunchKernelGGL(maxpool_to_nhwc_kernel<LQ_U8>, grid, dim3(256), lds, st, a);
    else hipLaunchKernelGGL(maxpool_to_nhwc_kernel<LQ_U8S8>, grid, dim3(256), lds, st, a);
    return launch_status(fn);
}

int lq_avgpool2d_global_nhwc(const int8_t* d_x, int x_type, const float* d_scale, const float* d_zero_point,
                             int64_t N, int64_t C, int64_t H, int64_t W, int x_pad, int64_t x_cs, float* d_y,
                             void* stream) {
    const char* fn = "lq_avgpool2d_global_nhwc";
    LQ_REQUIRE(x_type == LQ_I8 || x_type == LQ_U8 || x_type == LQ_U8S8, std::string(fn) + ": byte codes expected");
    LQ_REQUIRE(N >= 0 && C >= 1 && H >= 1 && W >= 1 && x_pad >= 0 && x_cs >= C && N * C < ((int64_t)1 << 31),
               std::string(fn) + ": bad shape");
    if (N == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y && d_scale, std::string(fn) + ": NULL pointer");
    const dim3 grid((unsigned)((N * C + AVG_NHWC_THREADS - 1) / AVG_NHWC_THREADS));
    const hipStream_t st = as_stream(stream);
#define LQ_AVG_NHWC(T_) hipLaunchKernelGGL(avgpool_global_nhwc_kernel<T_>, grid, dim3(AVG_NHWC_THREADS), 0, st, d_x, \
                                           N, (int)C, \
                                           (int)H, (int)W, x_pad, (int)x_cs, d_scale, d_zero_point, d_y)
    if (x_type == LQ_I8) LQ_AVG_NHWC(LQ_I8);
    else if (x_type == LQ_U8) LQ_AVG_NHWC(LQ_U8);
    else LQ_AVG_NHWC(LQ_U8S8);
#undef LQ_AVG_NHWC
    return launch_status(fn);
}

int lq_maxpool2d_i8_nhwc(const int8_t* d_x, int x_type, const float* d_zero_point, int64_t N, int64_t C, int64_t H,
                         int64_t W, int x_pad, int64_t x_cs, int64_t OH, int64_t OW, int KH, int KW, int stride_h,
                         int stride_w, int pad_h, int pad_w, int8_t* d_y, int y_pad, int64_t y_cs, void* stream) {
    const char* fn = "lq_maxpool2d_i8_nhwc";
    LQ_REQUIRE(x_type == LQ_I8 || x_type == LQ_U8 || x_type == LQ_U8S8, std::string(fn) + ": byte codes expected");
    LQ_REQUIRE(N >= 0 && C >= 16 && C % 16 == 0 && H >= 1 && W >= 1 && KH >= 1 && KW >= 1 && KH <= MPN_MAX_K &&
                   KW <= MPN_MAX_K && stride_h >= 1 && stride_w >= 1 && pad_h >= 0 && pad_w >= 0 &&
                   2 * pad_h <= KH && 2 * pad_w <= KW && x_pad >= 0 && x_cs >= C && x_cs % 16 == 0 && y_cs >= C &&
                   y_cs % 16 == 0 && y_pad >= 0 && y_pad <= 1,
               std::string(fn) + ": bad shape (C and the channel strides multiples of 16, windows up to 3 x 3)");
    LQ_REQUIRE(OH == (H + 2 * pad_h - KH) / stride_h + 1 && OW == (W + 2 * pad_w - KW) / stride_w + 1 &&
                   H + 2 * pad_h >= KH && W + 2 * pad_w >= KW,
               std::string(fn) + ": output size does not match the window");
    if (N == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y && d_zero_point && ((reinterpret_cast<uintptr_t>(d_x) | reinterpret_cast<uintptr_t>(d_y)) & 15) == 0,
               std::string(fn) + ": NULL or unaligned pointer");
    MaxNhwc2Args a{d_x, (int)N, (int)C, (int)H, (int)W, x_pad, (int)x_cs, (int)OH, (int)OW, KH, KW, stride_h,
                   stride_w, pad_h, pad_w, d_y, y_pad, (int)y_cs, d_zero_point};
    const int64_t total = N * OH * OW * (C / 16);
    const dim3 grid((unsigned)((total + 255) / 256));
    const hipStream_t st = as_stream(stream);
    if (x_type == LQ_I8) hipLaunchKernelGGL(maxpool_nhwc_kernel<LQ_I8>, grid, dim3(256), 0, st, a);
    else if (x_type == LQ_U8) hipLaunchKernelGGL(maxpool_nhwc_kernel<LQ_U8>, grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(maxpool_nhwc_kernel<LQ_U8S8>, grid, dim3(256), 0, st, a);
    return launch_status(fn);
}

}  // extern "C"
