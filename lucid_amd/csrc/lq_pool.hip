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

}  // extern "C"
