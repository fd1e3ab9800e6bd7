// lq_quant.hip -- bandwidth-bound kernels of the quantized path on gfx950:
// min/max observers, calculate_qparams, quantize, dequantize and fake-quantize.
//
// Reference compute each kernel replaces (lucid-official/lucid):
//   observers     observer.py:408-414 (MinMax), 527-544 (EMA), 672-685 (per channel),
//                 1031-1048 (per-channel EMA); NaN-propagating min/max Reduce.cpp:54-135
//   qparams       quantization/_qparams.py:186-205
//   quantize      quantization/_functional.py:59-69,179-197 (five Accelerate passes)
//   dequantize    quantization/_functional.py:281-293 (three passes)
//   fake-quant    quantization/_functional.py:314-333 (about ten passes incl. the mask)
// Here each is one pass: 128-bit loads and stores, 16 elements per lane, results
// identical bit-for-bit to the one-op-per-pass composition (no FMA contraction).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "lq_internal.h"

namespace lq {

constexpr int kBlock = 256;
constexpr int kVec = 16;  // elements per lane in the vector paths

// ------------------------------------------------------------ qparam sources
// A per-tensor parameter is either a device scalar (a Lucid tensor scale: its
// reciprocal is the float32 division 1.0f / s) or a host value passed by value
// (a Python-float scale: its reciprocal was rounded on the host from a double).
struct PtParams {
    const float* d_scale;
    const float* d_zp;
    float inv_value;
    float scale_value;
    float zp_value;
    __device__ __forceinline__ void load(float& inv, float& s, float& z) const {
        if (d_scale) {
            s = d_scale[0];
            inv = 1.0f / s;
        } else {
            inv = inv_value;
            s = scale_value;
        }
        z = d_zp ? d_zp[0] : zp_value;
    }
};

// ----------------------------------------------------------------- observers


// Block-wide min/max of keys; result valid in thread 0.
__device__ __forceinline__ void block_reduce_keys(int32_t& kmin, int32_t& kmax) {
    __shared__ int32_t smin[kBlock / 64], smax[kBlock / 64];
    kmin = wave_min(kmin);
    kmax = wave_max(kmax);
    int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    if (lane == 0) {
        smin[wid] = kmin;
        smax[wid] = kmax;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) {
            kmin = min(kmin, smin[w]);
            kmax = max(kmax, smax[w]);
        }
    }
}

// Stage 1: per-block extrema keys of x[n]; each block reduces one contiguous run of vf4 quads.
__global__ __launch_bounds__(kBlock) void minmax_partial_kernel(const float* __restrict__ x,
                                                                int64_t n, int2* __restrict__ part,
                                                                bool vec_ok) {
    int32_t kmin = KEY_POS_INF, kmax = KEY_NEG_INF;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t nthreads = (int64_t)gridDim.x * blockDim.x;
    int64_t done = 0;
    if (vec_ok) {
        const vf4* x4 = reinterpret_cast<const vf4*>(x);
        const int64_t nq = n >> 2;
        // This block's contiguous run of quads (a multiple of the block size), so each CU
        // streams one address range; four independent 128-bit loads in flight per lane.
        const int64_t bs = blockDim.x;
        const int64_t chunk = ((nq + gridDim.x - 1) / gridDim.x + bs - 1) / bs * bs;
        const int64_t b0 = min(nq, (int64_t)blockIdx.x * chunk), b1 = min(nq, b0 + chunk);
        int64_t i = b0 + threadIdx.x;
        for (; i + 3 * bs < b1; i += 4 * bs) {
            vf4 a = __builtin_nontemporal_load(&x4[i]);
            vf4 b = __builtin_nontemporal_load(&x4[i + bs]);
            vf4 c = __builtin_nontemporal_load(&x4[i + 2 * bs]);
            vf4 d = __builtin_nontemporal_load(&x4[i + 3 * bs]);
            key_accum(kmin, kmax, a.x); key_accum(kmin, kmax, a.y);
            key_accum(kmin, kmax, a.z); key_accum(kmin, kmax, a.w);
            key_accum(kmin, kmax, b.x); key_accum(kmin, kmax, b.y);
            key_accum(kmin, kmax, b.z); key_accum(kmin, kmax, b.w);
            key_accum(kmin, kmax, c.x); key_accum(kmin, kmax, c.y);
            key_accum(kmin, kmax, c.z); key_accum(kmin, kmax, c.w);
            key_accum(kmin, kmax, d.x); key_accum(kmin, kmax, d.y);
            key_accum(kmin, kmax, d.z); key_accum(kmin, kmax, d.w);
        }
        for (; i < b1; i += bs) {
            vf4 a = x4[i];
            key_accum(kmin, kmax, a.x); key_accum(kmin, kmax, a.y);
            key_accum(kmin, kmax, a.z); key_accum(kmin, kmax, a.w);
        }
        done = nq << 2;
    }
    for (int64_t i = done + tid; i < n; i += nthreads) key_accum(kmin, kmax, x[i]);
    block_reduce_keys(kmin, kmax);
    if (threadIdx.x == 0) part[blockIdx.x] = make_int2(kmin, kmax);
}

// Decode an extrema key pair: NaN in the data (keyed outside [-inf, +inf]) makes both NaN.

// Fold batch extrema into a running pair by mode (observer.py:408-414, 527-544).
__device__ __forceinline__ void fold_running(float& rmin, float& rmax, float cmin, float cmax,
                                             int mode, float c, bool first) {
    if (mode == LQ_OBS_REPLACE) {
        rmin = cmin;
        rmax = cmax;
    } else if (mode == LQ_OBS_MINMAX) {
        rmin = extreme_min(rmin, cmin);
        rmax = extreme_max(rmax, cmax);
    } else {
        if (first) {
            rmin = cmin;
            rmax = cmax;
        } else {
            float dmin = cmin - rmin;
            float dmax = cmax - rmax;
            float tmin = c * dmin;
            float tmax = c * dmax;
            rmin = rmin + tmin;
            rmax = rmax + tmax;
        }
    }
}

// Stage 2: one block folds the partials into the running {min, max}.
__global__ __launch_bounds__(kBlock) void minmax_finalize_kernel(const int2* __restrict__ part,
                                                                 int nparts, float* rmin_p,
                                                                 float* rmax_p, int mode, float c) {
    int32_t kmin = KEY_POS_INF, kmax = KEY_NEG_INF;
    for (int i = threadIdx.x; i < nparts; i += blockDim.x) {
        int2 p = part[i];
        kmin = min(kmin, p.x);
        kmax = max(kmax, p.y);
    }
    block_reduce_keys(kmin, kmax);
    if (threadIdx.x == 0) {
        float cmin, cmax;
        decode_keys(kmin, kmax, cmin, cmax);
        float rmin = *rmin_p, rmax = *rmax_p;
        bool first = __builtin_isinf(rmin);
        fold_running(rmin, rmax, cmin, cmax, mode, c, first);
        *rmin_p = rmin;
        *rmax_p = rmax;
    }
}

static int minmax_grid(int64_t n) {
    int64_t g = (n + (int64_t)kBlock * kVec - 1) / ((int64_t)kBlock * kVec);
    if (g < 1) g = 1;
    if (g > 4096) g = 4096;
    return (int)g;
}

// ---- per channel, x as [outer, C, inner]
// Row form (inner >= 64): block (c, split) reduces channel c over its share of `outer`.
__global__ __launch_bounds__(kBlock) void minmax_pc_rows_kernel(const float* __restrict__ x,
                                                                int64_t outer, int64_t C,
                                                                int64_t inner, int splits,
                                                                int2* __restrict__ part,
                                                                bool vec_ok) {
    const int64_t c = blockIdx.x;
    const int split = blockIdx.y;
    int32_t kmin = KEY_POS_INF, kmax = KEY_NEG_INF;
    for (int64_t o = split; o < outer; o += splits) {
        const float* row = x + (o * C + c) * inner;
        int64_t done = 0;
        if (vec_ok) {
            const vf4* r4 = reinterpret_cast<const vf4*>(row);
            const int64_t nq = inner >> 2;
            int64_t i = threadIdx.x;
            for (; i + 3 * kBlock < nq; i += 4 * kBlock) {
                vf4 a = __builtin_nontemporal_load(&r4[i]);
                vf4 b = __builtin_nontemporal_load(&r4[i + kBlock]);
                vf4 cc = __builtin_nontemporal_load(&r4[i + 2 * kBlock]);
                vf4 d = __builtin_nontemporal_load(&r4[i + 3 * kBlock]);
                key_accum(kmin, kmax, a.x); key_accum(kmin, kmax, a.y);
                key_accum(kmin, kmax, a.z); key_accum(kmin, kmax, a.w);
                key_accum(kmin, kmax, b.x); key_accum(kmin, kmax, b.y);
                key_accum(kmin, kmax, b.z); key_accum(kmin, kmax, b.w);
                key_accum(kmin, kmax, cc.x); key_accum(kmin, kmax, cc.y);
                key_accum(kmin, kmax, cc.z); key_accum(kmin, kmax, cc.w);
                key_accum(kmin, kmax, d.x); key_accum(kmin, kmax, d.y);
                key_accum(kmin, kmax, d.z); key_accum(kmin, kmax, d.w);
            }
            for (; i < nq; i += kBlock) {
                vf4 a = r4[i];
                key_accum(kmin, kmax, a.x); key_accum(kmin, kmax, a.y);
                key_accum(kmin, kmax, a.z); key_accum(kmin, kmax, a.w);
            }
            done = nq << 2;
        }
        for (int64_t i = done + threadIdx.x; i < inner; i += kBlock) key_accum(kmin, kmax, row[i]);
    }
    block_reduce_keys(kmin, kmax);
    if (threadIdx.x == 0) part[(int64_t)split * C + c] = make_int2(kmin, kmax);
}

// Column form (inner < 64): lane j of block (tile, split) owns column j of the
// [outer, C*inner] matrix and walks its share of the rows (coalesced across lanes).
__global__ __launch_bounds__(kBlock) void minmax_pc_cols_kernel(const float* __restrict__ x,
                                                                int64_t outer, int64_t width,
                                                                int splits,
                                                                int2* __restrict__ part) {
    const int64_t j = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const int split = blockIdx.y;
    if (j >= width) return;
    int32_t kmin = KEY_POS_INF, kmax = KEY_NEG_INF;
    for (int64_t o = split; o < outer; o += splits) key_accum(kmin, kmax, x[o * width + j]);
    part[(int64_t)split * width + j] = make_int2(kmin, kmax);
}

// Fold per-channel partials: part is [splits, C * per_c] key pairs (per_c = inner for the
// column form, 1 for the row form).  One block; the per-channel EMA seed test reads the
// whole running_min first (observer.py:1039-1044).
__global__ __launch_bounds__(1024) void minmax_pc_finalize_kernel(const int2* __restrict__ part,
                                                                  int splits, int64_t C,
                                                                  int64_t per_c, float* rmin,
                                                                  float* rmax, int mode,
                                                                  float c) {
    __shared__ int all_inf;
    if (threadIdx.x == 0) all_inf = 1;
    __syncthreads();
    if (mode == LQ_OBS_EMA) {
        for (int64_t ch = threadIdx.x; ch < C; ch += blockDim.x)
            if (!__builtin_isinf(rmin[ch])) all_inf = 0;  // benign race: all writers store 0
        __syncthreads();
    }
    const bool first = all_inf != 0;
    for (int64_t ch = threadIdx.x; ch < C; ch += blockDim.x) {
        int32_t kmin = KEY_POS_INF, kmax = KEY_NEG_INF;
        for (int s = 0; s < splits; ++s)
            for (int64_t i = 0; i < per_c; ++i) {
                int2 p = part[(int64_t)s * C * per_c + ch * per_c + i];
                kmin = min(kmin, p.x);
                kmax = max(kmax, p.y);
            }
        float cmin, cmax;
        decode_keys(kmin, kmax, cmin, cmax);
        float a = rmin[ch], b = rmax[ch];
        fold_running(a, b, cmin, cmax, mode, c, first);
        rmin[ch] = a;
        rmax[ch] = b;
    }
}

struct PcPlan {
    bool rows;
    int splits;
    int64_t per_c;
    size_t bytes;
};

static PcPlan pc_plan(int64_t outer, int64_t C, int64_t inner) {
    PcPlan p;
    p.rows = inner >= 64;
    if (p.rows) {
        // Enough blocks to fill the chip, each with at least ~16K elements.
        int64_t want = (C >= 1024) ? 1 : (1024 + C - 1) / C;
        int64_t max_by_work = (outer * inner) / 16384;
        if (want > max_by_work) want = max_by_work;
        if (want > outer) want = outer;
        if (want < 1) want = 1;
        p.splits = (int)want;
        p.per_c = 1;
        p.bytes = sizeof(int2) * (size_t)(p.splits * C);
    } else {
        int64_t width = C * inner;
        int64_t tiles = (width + kBlock - 1) / kBlock;
        int64_t want = (tiles >= 1024 || tiles == 0) ? 1 : (1024 + tiles - 1) / tiles;
        int64_t max_by_work = outer / 64;
        if (want > max_by_work) want = max_by_work;
        if (want < 1) want = 1;
        p.splits = (int)want;
        p.per_c = inner;
        p.bytes = sizeof(int2) * (size_t)(p.splits * width);
    }
    return p;
}

// ------------------------------------------------------------------ qparams
// calculate_qparams (_qparams.py:186-205), one lane per range.
__global__ void calc_qparams_kernel(const float* __restrict__ mn_in, const float* __restrict__ mx_in,
                                    int64_t n, int symmetric, int is_signed, int qmin, int qmax,
                                    float eps, float* __restrict__ scale,
                                    float* __restrict__ zero_point, float half_range,
                                    float width_f, float mid_zp, Grid g) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float mn = extreme_min(mn_in[i], 0.0f);  // lucid.minimum(min, zeros_like)
    float mx = extreme_max(mx_in[i], 0.0f);
    if (symmetric) {
        float ma = extreme_max(__builtin_fabsf(mn), __builtin_fabsf(mx));
        float q = ma / half_range;
        scale[i] = extreme_max(q, eps);
        zero_point[i] = is_signed ? 0.0f : mid_zp;
    } else {
        float w = mx - mn;
        float q = w / width_f;
        float s = extreme_max(q, eps);
        float r = rne(mn / s);
        float z = (float)qmin - r;
        scale[i] = s;
        zero_point[i] = clip_grid(z, g);
    }
}

// -------------------------------------------------------- quantize kernels

template <class Code, int N>
struct CodeVec {
    typename Code::T v[N];
};


template <class Code>
__device__ __forceinline__ void store16(typename Code::T* dst, const float* c) {
    CodeVec<Code, kVec> out;
#pragma unroll
    for (int j = 0; j < kVec; ++j) out.v[j] = Code::store(c[j]);
    constexpr int bytes = sizeof(out);
    static_assert(bytes % 16 == 0, "16-element code vector is a multiple of 16 bytes");
    const vu4* s = reinterpret_cast<const vu4*>(&out);
    vu4* d = reinterpret_cast<vu4*>(dst);
#pragma unroll
    for (int j = 0; j < bytes / 16; ++j) __builtin_nontemporal_store(s[j], &d[j]);
}

__device__ __forceinline__ void load16(const float* src, float* v) {
    const vf4* s = reinterpret_cast<const vf4*>(src);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        vf4 a = __builtin_nontemporal_load(&s[j]);
        v[4 * j + 0] = a.x;
        v[4 * j + 1] = a.y;
        v[4 * j + 2] = a.z;
        v[4 * j + 3] = a.w;
    }
}

// Per-tensor: lane t handles elements [16t, 16t+16) when the vector path applies.
template <class Code>
__global__ __launch_bounds__(kBlock) void quantize_pt_kernel(const float* __restrict__ x,
                                                             typename Code::T* __restrict__ q,
                                                             int64_t n, PtParams pp, Grid g,
                                                             bool vec_ok) {
    float inv, s, z;
    pp.load(inv, s, z);
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (vec_ok) {
        const int64_t base = t * kVec;
        if (base + kVec <= n) {
            float v[kVec], c[kVec];
            load16(x + base, v);
#pragma unroll
            for (int j = 0; j < kVec; ++j) c[j] = quant_one<Code>(v[j], inv, z, g);
            store16<Code>(q + base, c);
        } else {
            for (int64_t i = base; i < n; ++i) q[i] = Code::store(quant_one<Code>(x[i], inv, z, g));
        }
    } else {
        const int64_t stride = (int64_t)gridDim.x * blockDim.x;
        for (int64_t i = t; i < n; i += stride) q[i] = Code::store(quant_one<Code>(x[i], inv, z, g));
    }
}

// Channel of flat element i in [outer, C, inner].
__device__ __forceinline__ int64_t channel_of(int64_t i, int64_t C, int64_t inner) {
    if (inner == 1) return i % C;
    return (i / inner) % C;
}

template <class Code>
__global__ __launch_bounds__(kBlock) void quantize_pc_kernel(
    const float* __restrict__ x, typename Code::T* __restrict__ q, int64_t n, int64_t C,
    int64_t inner, const float* __restrict__ scale, const float* __restrict__ zp, float zp_value,
    Grid g, bool vec_ok) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (vec_ok) {  // inner % 16 == 0: the 16 elements share one channel
        const int64_t base = t * kVec;
        if (base >= n) return;
        const int64_t ch = channel_of(base, C, inner);
        const float inv = 1.0f / scale[ch];
        const float z = zp ? zp[ch] : zp_value;
        float v[kVec], c[kVec];
        load16(x + base, v);
#pragma unroll
        for (int j = 0; j < kVec; ++j) c[j] = quant_one<Code>(v[j], inv, z, g);
        store16<Code>(q + base, c);
    } else {
        const int64_t stride = (int64_t)gridDim.x * blockDim.x;
        for (int64_t i = t; i < n; i += stride) {
            const int64_t ch = channel_of(i, C, inner);
            const float inv = 1.0f / scale[ch];
            const float z = zp ? zp[ch] : zp_value;
            q[i] = Code::store(quant_one<Code>(x[i], inv, z, g));
        }
    }
}

// ------------------------------------------------------- dequantize kernels

template <typename Y>
__device__ __forceinline__ Y to_out(float v);
template <>
__device__ __forceinline__ float to_out<float>(float v) { return v; }
template <>
__device__ __forceinline__ __half to_out<__half>(float v) { return f32_to_f16_rn(v); }

template <class Code, typename Y>
__device__ __forceinline__ void dequant16(const typename Code::T* src, Y* dst, float s, float z) {
    CodeVec<Code, kVec> in;
    constexpr int inb = sizeof(in);
    const vu4* sp = reinterpret_cast<const vu4*>(src);
    vu4* ip = reinterpret_cast<vu4*>(&in);
#pragma unroll
    for (int j = 0; j < inb / 16; ++j) ip[j] = __builtin_nontemporal_load(&sp[j]);
    Y out[kVec];
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
        float f = Code::load(in.v[j]);
        float d = f - z;
        out[j] = to_out<Y>(d * s);
    }
    constexpr int outb = sizeof(out);
    const vu4* op = reinterpret_cast<const vu4*>(out);
    vu4* dp = reinterpret_cast<vu4*>(dst);
#pragma unroll
    for (int j = 0; j < outb / 16; ++j) __builtin_nontemporal_store(op[j], &dp[j]);
}

template <class Code, typename Y>
__global__ __launch_bounds__(kBlock) void dequantize_pt_kernel(const typename Code::T* __restrict__ q,
                                                               Y* __restrict__ y, int64_t n,
                                                               PtParams pp, bool vec_ok) {
    float inv, s, z;
    pp.load(inv, s, z);
    (void)inv;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (vec_ok) {
        const int64_t base = t * kVec;
        if (base + kVec <= n) {
            dequant16<Code, Y>(q + base, y + base, s, z);
        } else {
            for (int64_t i = base; i < n; ++i) {
                float d = Code::load(q[i]) - z;
                y[i] = to_out<Y>(d * s);
            }
        }
    } else {
        const int64_t stride = (int64_t)gridDim.x * blockDim.x;
        for (int64_t i = t; i < n; i += stride) {
            float d = Code::load(q[i]) - z;
            y[i] = to_out<Y>(d * s);
        }
    }
}

template <class Code, typename Y>
__global__ __launch_bounds__(kBlock) void dequantize_pc_kernel(
    const typename Code::T* __restrict__ q, Y* __restrict__ y, int64_t n, int64_t C, int64_t inner,
    const float* __restrict__ scale, const float* __restrict__ zp, float zp_value, bool vec_ok) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (vec_ok) {
        const int64_t base = t * kVec;
        if (base >= n) return;
        const int64_t ch = channel_of(base, C, inner);
        dequant16<Code, Y>(q + base, y + base, scale[ch], zp ? zp[ch] : zp_value);
    } else {
        const int64_t stride = (int64_t)gridDim.x * blockDim.x;
        for (int64_t i = t; i < n; i += stride) {
            const int64_t ch = channel_of(i, C, inner);
            float d = Code::load(q[i]) - (zp ? zp[ch] : zp_value);
            y[i] = to_out<Y>(d * scale[ch]);
        }
    }
}

// ---------------------------------------------------- fake-quantize kernels

__device__ __forceinline__ float fq_one(float x, float inv, float s, float z, const Grid& g,
                                        float& m) {
    float t = x * inv;
    float r = rne(t);
    float qpre = r + z;
    float qc = clip_grid(qpre, g);
    float d = qc - z;
    float lo = (qpre >= g.lo) ? 1.0f : 0.0f;
    float hi = (qpre <= g.hi) ? 1.0f : 0.0f;
    m = lo * hi;
    return d * s;
}

__device__ __forceinline__ void store16f(float* dst, const float* v) {
    vf4* d = reinterpret_cast<vf4*>(dst);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        __builtin_nontemporal_store(vf4{v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]}, &d[j]);
}

__global__ __launch_bounds__(kBlock) void fake_quant_kernel(const float* __restrict__ x,
                                                            float* __restrict__ y,
                                                            float* __restrict__ mask, int64_t n,
                                                            int64_t C, int64_t inner, PtParams pp,
                                                            const float* __restrict__ scale,
                                                            const float* __restrict__ zp,
                                                            float zp_value, Grid g, bool per_channel,
                                                            bool vec_ok) {
    float inv = 0.f, s = 0.f, z = 0.f;
    if (!per_channel) pp.load(inv, s, z);
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (vec_ok) {
        const int64_t base = t * kVec;
        if (base + kVec <= n) {
            if (per_channel) {
                const int64_t ch = channel_of(base, C, inner);
                s = scale[ch];
                inv = 1.0f / s;
                z = zp ? zp[ch] : zp_value;
            }
            float v[kVec], o[kVec], m[kVec];
            load16(x + base, v);
#pragma unroll
            for (int j = 0; j < kVec; ++j) o[j] = fq_one(v[j], inv, s, z, g, m[j]);
            store16f(y + base, o);
            if (mask) store16f(mask + base, m);
            return;
        }
        for (int64_t i = base; i < n; ++i) {
            if (per_channel) {
                const int64_t ch = channel_of(i, C, inner);
                s = scale[ch];
                inv = 1.0f / s;
                z = zp ? zp[ch] : zp_value;
            }
            float m;
            y[i] = fq_one(x[i], inv, s, z, g, m);
            if (mask) mask[i] = m;
        }
    } else {
        const int64_t stride = (int64_t)gridDim.x * blockDim.x;
        for (int64_t i = t; i < n; i += stride) {
            if (per_channel) {
                const int64_t ch = channel_of(i, C, inner);
                s = scale[ch];
                inv = 1.0f / s;
                z = zp ? zp[ch] : zp_value;
            }
            float m;
            y[i] = fq_one(x[i], inv, s, z, g, m);
            if (mask) mask[i] = m;
        }
    }
}

// ------------------------------------------------ grouped (4-wide) vector kernels
//
// The aligned path of quantize / dequantize / fake-quantize.  Work is split into groups of
// four consecutive elements, and every memory instruction is contiguous across the lanes
// of a wave: float groups move as 16-byte vectors, code groups as 4 / 8 / 16-byte vectors
// (1 / 2 / 4-byte codes).  Each block walks its own contiguous run of groups, each thread
// keeping four groups in flight.  Qparams: per tensor (PT), one channel per group (PCG, inner % 4 == 0) or a
// channel per element (PCE).  Elements past the last whole group are handled one by one.

enum { PT = 0, PCG = 1, PCE = 2 };
constexpr int kGrpUnroll = 4;

template <int BYTES> struct RawVec;
template <> struct RawVec<4> { typedef uint32_t T; };
template <> struct RawVec<8> { typedef uint32_t T __attribute__((ext_vector_type(2))); };
template <> struct RawVec<16> { typedef vu4 T; };

template <class Code>
struct Group4 {
    typedef typename Code::T T;
    typedef typename RawVec<4 * sizeof(T)>::T Raw;
    union U {
        Raw raw;
        T v[4];
    };
};

// Channel of element e of an [outer, C, inner] tensor (32-bit indices: n < 2^32).
__device__ __forceinline__ uint32_t chan_of(uint32_t e, uint32_t C, uint32_t inner) {
    return (e / inner) % C;
}

struct QArgs {
    const float* d_scale;  // per tensor: [1] or NULL (then inv_value / scale_value); per channel: [C]
    const float* d_zp;     // [1] / [C] or NULL (then zp_value)
    float inv_value, scale_value, zp_value;
    uint32_t C, inner;
    __device__ __forceinline__ void tensor(float& inv, float& s, float& z) const {
        if (d_scale) {
            s = d_scale[0];
            inv = 1.0f / s;
        } else {
            inv = inv_value;
            s = scale_value;
        }
        z = d_zp ? d_zp[0] : zp_value;
    }
    __device__ __forceinline__ void channel(uint32_t c, float& inv, float& s, float& z) const {
        s = d_scale[c];
        inv = 1.0f / s;
        z = d_zp ? d_zp[c] : zp_value;
    }
};

template <int MODE>
__device__ __forceinline__ void group_params(const QArgs& q, uint32_t e0, int j, float t_inv, float t_s,
                                             float t_z, float& inv, float& s, float& z) {
    if (MODE == PT) {
        inv = t_inv;
        s = t_s;
        z = t_z;
    } else {
        q.channel(chan_of(e0 + (MODE == PCE ? j : 0), q.C, q.inner), inv, s, z);
    }
}

// Block-contiguous share of [0, n) groups: block b owns one run of consecutive groups (a
// multiple of kBlock) and its lanes walk it kBlock apart, so each CU streams its own
// contiguous address range (on MI355X a 1 GB read stream runs at ~7.0 TB/s this way,
// against 5.6-6.1 TB/s grid-stride over the whole tensor).
struct BlockRun {
    uint32_t i, end;
};
__device__ __forceinline__ BlockRun block_run(uint32_t n) {
    const uint32_t chunk = ((n + gridDim.x - 1) / gridDim.x + kBlock - 1) / kBlock * kBlock;
    const uint32_t b = min(n, blockIdx.x * chunk);
    return BlockRun{b + threadIdx.x, min(n, b + chunk)};
}

// One group of four codes of quantize_g4_kernel.
template <class Code, int MODE>
__device__ __forceinline__ void quantize_group4(typename Group4<Code>::Raw* __restrict__ q4, uint32_t gi, vf4 v,
                                                const QArgs& qa, Grid g, float t_inv, float t_s, float t_z) {
    typename Group4<Code>::U o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float inv, s, z;
        group_params<MODE>(qa, gi * 4, j, t_inv, t_s, t_z, inv, s, z);
        o.v[j] = quant_store<Code>(v[j], inv, z, g);
    }
    q4[gi] = o.raw;
}

constexpr int kG4Inflight = 4 * kGrpUnroll;  // groups in flight per lane

// The body of quantize_g4_kernel with the per-tensor parameters (t_inv, t_s, t_z) given; the
// lane's first `skip` groups (0 or kG4Inflight) have been quantized by the caller.
template <class Code, int MODE>
__device__ __forceinline__ void quantize_g4_run(const float* __restrict__ x, typename Code::T* __restrict__ q,
                                                uint32_t n, const QArgs& qa, Grid g, float t_inv, float t_s,
                                                float t_z, uint32_t skip = 0) {
    typedef Group4<Code> G;
    const uint32_t ng = n >> 2;
    const vf4* x4 = reinterpret_cast<const vf4*>(x);
    typename G::Raw* q4 = reinterpret_cast<typename G::Raw*>(q);
    // Streaming reads bypass the caches (nontemporal); the 4x smaller code stores do not.
    // Sixteen groups in flight per lane (with up to 8192 workgroups): the per-element rounding
    // and clipping would otherwise leave too few loads outstanding to cover HBM latency
    // (measured on 2^28 floats: 8 groups x 4096 workgroups 72-75%, 16 x 8192 77-79% of peak).
    constexpr int U = kG4Inflight;
    const BlockRun r = block_run(ng);
    uint32_t i = r.i + skip * kBlock;
    for (; i + (U - 1) * kBlock < r.end; i += U * kBlock) {
        vf4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(&x4[i + u * kBlock]);
#pragma unroll
        for (int u = 0; u < U; ++u) quantize_group4<Code, MODE>(q4, i + u * kBlock, v[u], qa, g, t_inv, t_s, t_z);
    }
    for (; i < r.end; i += kBlock)
        quantize_group4<Code, MODE>(q4, i, __builtin_nontemporal_load(&x4[i]), qa, g, t_inv, t_s, t_z);
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        const uint32_t e = ng * 4 + threadIdx.x;
        float inv, s, z;
        if (MODE == PT) {
            inv = t_inv;
            z = t_z;
        } else {
            qa.channel(chan_of(e, qa.C, qa.inner), inv, s, z);
        }
        q[e] = Code::store(quant_one<Code>(x[e], inv, z, g));
    }
}

template <class Code, int MODE>
__global__ __launch_bounds__(kBlock) void quantize_g4_kernel(const float* __restrict__ x,
                                                             typename Code::T* __restrict__ q,
                                                             uint32_t n, QArgs qa, Grid g) {
    float t_inv = 0.f, t_s = 0.f, t_z = 0.f;
    if (MODE == PT) qa.tensor(t_inv, t_s, t_z);
    quantize_g4_run<Code, MODE>(x, q, n, qa, g, t_inv, t_s, t_z);
}

template <class Code, typename Y, int MODE>
__global__ __launch_bounds__(kBlock) void dequantize_g4_kernel(const typename Code::T* __restrict__ q,
                                                               Y* __restrict__ y, uint32_t n, QArgs qa) {
    typedef Group4<Code> G;
    typedef typename RawVec<4 * sizeof(Y)>::T YRaw;
    union YU {
        YRaw raw;
        Y v[4];
    };
    const uint32_t ng = n >> 2;
    float t_inv = 0.f, t_s = 0.f, t_z = 0.f;
    if (MODE == PT) qa.tensor(t_inv, t_s, t_z);
    const typename G::Raw* q4 = reinterpret_cast<const typename G::Raw*>(q);
    YRaw* y4 = reinterpret_cast<YRaw*>(y);
    auto one = [&](uint32_t gi, typename G::Raw raw) __attribute__((always_inline)) {
        typename G::U in;
        in.raw = raw;
        YU o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float inv, s, z;
            group_params<MODE>(qa, gi * 4, j, t_inv, t_s, t_z, inv, s, z);
            const float d = Code::load(in.v[j]) - z;
            o.v[j] = to_out<Y>(d * s);
        }
        __builtin_nontemporal_store(o.raw, &y4[gi]);
    };
    // The small code reads stay cached; the 4x larger float stores are nontemporal.
    const BlockRun br = block_run(ng);
    uint32_t i = br.i;
    for (; i + (kGrpUnroll - 1) * kBlock < br.end; i += kGrpUnroll * kBlock) {
        typename G::Raw r[kGrpUnroll];
#pragma unroll
        for (int u = 0; u < kGrpUnroll; ++u) r[u] = q4[i + u * kBlock];
#pragma unroll
        for (int u = 0; u < kGrpUnroll; ++u) one(i + u * kBlock, r[u]);
    }
    for (; i < br.end; i += kBlock) one(i, q4[i]);
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        const uint32_t e = ng * 4 + threadIdx.x;
        float inv, s, z;
        if (MODE == PT) {
            s = t_s;
            z = t_z;
        } else {
            qa.channel(chan_of(e, qa.C, qa.inner), inv, s, z);
        }
        const float d = Code::load(q[e]) - z;
        y[e] = to_out<Y>(d * s);
    }
}

template <int MODE, bool MASK>
__global__ __launch_bounds__(kBlock) void fake_quant_g4_kernel(const float* __restrict__ x,
                                                               float* __restrict__ y,
                                                               float* __restrict__ mask, uint32_t n,
                                                               QArgs qa, Grid g) {
    const uint32_t ng = n >> 2;
    float t_inv = 0.f, t_s = 0.f, t_z = 0.f;
    if (MODE == PT) qa.tensor(t_inv, t_s, t_z);
    const vf4* x4 = reinterpret_cast<const vf4*>(x);
    vf4* y4 = reinterpret_cast<vf4*>(y);
    vf4* m4 = reinterpret_cast<vf4*>(mask);
    auto one = [&](uint32_t gi, vf4 v) __attribute__((always_inline)) {
        vf4 o, mk;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float inv, s, z, m;
            group_params<MODE>(qa, gi * 4, j, t_inv, t_s, t_z, inv, s, z);
            o[j] = fq_one(v[j], inv, s, z, g, m);
            mk[j] = m;
        }
        __builtin_nontemporal_store(o, &y4[gi]);
        if (MASK) __builtin_nontemporal_store(mk, &m4[gi]);
    };
    const BlockRun br = block_run(ng);
    uint32_t i = br.i;
    for (; i + (kGrpUnroll - 1) * kBlock < br.end; i += kGrpUnroll * kBlock) {
        vf4 v[kGrpUnroll];
#pragma unroll
        for (int u = 0; u < kGrpUnroll; ++u) v[u] = x4[i + u * kBlock];
#pragma unroll
        for (int u = 0; u < kGrpUnroll; ++u) one(i + u * kBlock, v[u]);
    }
    for (; i < br.end; i += kBlock) one(i, x4[i]);
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        const uint32_t e = ng * 4 + threadIdx.x;
        float inv, s, z, m;
        if (MODE == PT) {
            inv = t_inv;
            s = t_s;
            z = t_z;
        } else {
            qa.channel(chan_of(e, qa.C, qa.inner), inv, s, z);
        }
        y[e] = fq_one(x[e], inv, s, z, g, m);
        if (MASK) mask[e] = m;
    }
}

// ------------------------------------------------------------------- launch helpers

// Grouped kernels: enough blocks to keep every CU streaming (16 blocks of 256 per CU),
// never more than one group per thread.
static dim3 g4_grid(int64_t n) {
    int64_t groups = (n + 3) / 4;
    int64_t blocks = (groups + kBlock - 1) / kBlock;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    return dim3((unsigned)blocks);
}

// The quantize stream keeps more workgroups resident (its loads are the latency to cover).
static dim3 g4_quant_grid(int64_t n) {
    int64_t groups = (n + 3) / 4;
    int64_t blocks = (groups + kBlock - 1) / kBlock;
    if (blocks > 8192) blocks = 8192;
    if (blocks < 1) blocks = 1;
    return dim3((unsigned)blocks);
}

static dim3 scalar_grid(int64_t n) {
    int64_t blocks = (n + kBlock - 1) / kBlock;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    return dim3((unsigned)blocks);
}

static bool valid_code(int t) {
    return t == LQ_I8 || t == LQ_U8 || t == LQ_I16 || t == LQ_I32 || t == LQ_U8S8;
}

template <template <class> class F, typename... Args>
static int dispatch_code(int q_dtype, Args&&... args) {
    switch (q_dtype) {
    case LQ_I8: return F<CodeI8>::run(args...);
    case LQ_U8: return F<CodeU8>::run(args...);
    case LQ_I16: return F<CodeI16>::run(args...);
    case LQ_I32: return F<CodeI32>::run(args...);
    case LQ_U8S8: return F<CodeU8S8>::run(args...);
    default: return set_error(LQ_ERR_INVALID, "unsupported code dtype");
    }
}

// Grouped path applies: 16-byte aligned float side, code side aligned for its group vector,
// 32-bit element indices.
template <class Code>
static bool g4_ok(const void* f, const void* c, int64_t n) {
    const uintptr_t ca = 4 * sizeof(typename Code::T) - 1;
    return aligned16(f) && ((reinterpret_cast<uintptr_t>(c) & ca) == 0) && n < ((int64_t)1 << 32);
}

static bool g4_ok_code(int q_dtype, const void* f, const void* c, int64_t n) {
    switch (q_dtype) {
    case LQ_I8: return g4_ok<CodeI8>(f, c, n);
    case LQ_U8: return g4_ok<CodeU8>(f, c, n);
    case LQ_I16: return g4_ok<CodeI16>(f, c, n);
    case LQ_I32: return g4_ok<CodeI32>(f, c, n);
    case LQ_U8S8: return g4_ok<CodeU8S8>(f, c, n);
    default: return false;
    }
}

// ------------------------------------------------- dynamic activation quantization
//
// The dynamic Linear's activation step (lucid/nn/quantized/dynamic/linear.py:85-92): the live
// range of x (MinMaxObserver, replace), per-tensor affine qparams from it (_qparams.py:186-205)
// and the quantize on that grid, in one launch of one workgroup for tensors up to
// DYN_SMALL_MAX elements (a decode step's rows).  The same device arithmetic as the
// separate launches: extrema as ordered integer keys (order-free), the asymmetric branch of
// calc_qparams_kernel, the reciprocal 1.0f / s and quant_one of the per-tensor quantize, so
// the scalars and codes are the same bits.
constexpr int64_t DYN_SMALL_MAX = 16384;  // above it, one workgroup is slower than three launches
constexpr int kDynBlock = 1024;

template <class Code>
__global__ __launch_bounds__(kDynBlock) void dyn_quant_small_kernel(const float* __restrict__ x, int n,
                                                                    typename Code::T* __restrict__ q,
                                                                    float* __restrict__ qp, int qmin, float eps,
                                                                    float width_f, Grid g, bool vec_ok) {
    __shared__ int32_t smin[kDynBlock / 64], smax[kDynBlock / 64];
    __shared__ float s_sz[2];
    const int tid = threadIdx.x;
    int32_t kmin = KEY_POS_INF, kmax = KEY_NEG_INF;
    const int nq = vec_ok ? (n >> 2) : 0;
    for (int i = tid; i < nq; i += kDynBlock) {
        const vf4 v = reinterpret_cast<const vf4*>(x)[i];
        key_accum(kmin, kmax, v.x);
        key_accum(kmin, kmax, v.y);
        key_accum(kmin, kmax, v.z);
        key_accum(kmin, kmax, v.w);
    }
    for (int i = 4 * nq + tid; i < n; i += kDynBlock) key_accum(kmin, kmax, x[i]);
    kmin = wave_min(kmin);
    kmax = wave_max(kmax);
    if ((tid & 63) == 0) {
        smin[tid >> 6] = kmin;
        smax[tid >> 6] = kmax;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kDynBlock / 64; ++w) {
            kmin = min(kmin, smin[w]);
            kmax = max(kmax, smax[w]);
        }
        float o[4];
        dyn_qparams(kmin, kmax, qmin, eps, width_f, g, o);
        qp[0] = o[0];
        qp[1] = o[1];
        qp[2] = o[2];
        qp[3] = o[3];
        s_sz[0] = o[2];
        s_sz[1] = o[3];
    }
    __syncthreads();
    const float sc = s_sz[0], z = s_sz[1];
    const float inv = 1.0f / sc;
    for (int i = tid; i < n; i += kDynBlock) q[i] = Code::store(quant_one<Code>(x[i], inv, z, g));
}

// Above DYN_SMALL_MAX, with aligned float and code vectors: two launches.  minmax_partial_kernel
// leaves at most DYN_PARTS_MAX extrema key pairs; every workgroup of dyn_quantize_g4_kernel
// folds all of them (min / max of keys: any order gives the same pair), derives the qparams
// with dyn_qparams and quantizes its run of groups as quantize_g4_kernel does with a device
// scale (inv = 1.0f / s) -- the bits of minmax, calc_qparams and the per-tensor quantize.
// Workgroup 0 stores {min, max, scale, zero point}.
static_assert(DYN_PARTS_MAX == 4 * kBlock, "four partials per lane in the fold");

// U: groups per lane read ahead, the launch's groups per lane rounded up to a power of two
// (at most kG4Inflight), so almost every early load is one the lane uses.
template <class Code, int U>
__global__ __launch_bounds__(kBlock) void dyn_quantize_g4_kernel(const float* __restrict__ x,
                                                                 typename Code::T* __restrict__ q, uint32_t n,
                                                                 const int2* __restrict__ part, int nparts,
                                                                 float* __restrict__ qp, int qmin, float eps,
                                                                 float width_f, Grid g) {
    typedef Group4<Code> G;
    __shared__ float s_sz[2];
    const BlockRun r = block_run(n >> 2);
    const vf4* x4 = reinterpret_cast<const vf4*>(x);
    // The partials, then the lane's first U groups, are read before the qparams exist: all
    // in flight together, so the fold costs no extra memory round trip.  Every load is
    // unconditional, its index wrapped or clamped into range (a repeated partial changes no
    // extremum, and wrapping spreads the repeats over the array instead of one hot line;
    // groups past the run are loaded but not used): with no branch between them the wait for
    // the partials leaves the group loads, issued after them, outstanding.
    int2 p[DYN_PARTS_MAX / kBlock];
#pragma unroll
    for (int u = 0; u < DYN_PARTS_MAX / kBlock; ++u) {
        const int i = (int)threadIdx.x + u * kBlock;
        p[u] = part[i < nparts ? i : i % nparts];
    }
    const uint32_t last = (n >> 2) - 1;  // n >= 4 on this path
    vf4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t i = r.i + u * kBlock;
        v[u] = __builtin_nontemporal_load(&x4[i < last ? i : last]);
    }
    int32_t kmin = p[0].x, kmax = p[0].y;
#pragma unroll
    for (int u = 1; u < DYN_PARTS_MAX / kBlock; ++u) {
        kmin = min(kmin, p[u].x);
        kmax = max(kmax, p[u].y);
    }
    block_reduce_keys(kmin, kmax);
    if (threadIdx.x == 0) {
        float o[4];
        dyn_qparams(kmin, kmax, qmin, eps, width_f, g, o);
        if (blockIdx.x == 0) {
            qp[0] = o[0];
            qp[1] = o[1];
            qp[2] = o[2];
            qp[3] = o[3];
        }
        s_sz[0] = o[2];
        s_sz[1] = o[3];
    }
    __syncthreads();
    const float s = s_sz[0], z = s_sz[1], inv = 1.0f / s;
    const QArgs qa{};
    typename G::Raw* q4 = reinterpret_cast<typename G::Raw*>(q);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t i = r.i + u * kBlock;
        if (i < r.end) quantize_group4<Code, PT>(q4, i, v[u], qa, g, inv, s, z);
    }
    quantize_g4_run<Code, PT>(x, q, n, qa, g, inv, s, z, U);
}

// At most 1024 workgroups (four per CU): each lane's first kG4Inflight groups, read before the
// qparams, cover the whole tensor up to 2^24 elements.
static dim3 dyn_g4_grid(int64_t n) {
    const dim3 g = g4_quant_grid(n);
    return dim3(g.x < 1024u ? g.x : 1024u);
}

// Groups per lane of block_run's split over `grid` workgroups, rounded up to a power of two.
static int dyn_g4_unroll(int64_t n, unsigned grid) {
    const int64_t ng = n >> 2;
    const int64_t chunk = ((ng + grid - 1) / grid + kBlock - 1) / kBlock * kBlock;
    const int64_t per = chunk / kBlock;
    int u = 1;
    while (u < per && u < kG4Inflight) u *= 2;
    return u;
}

template <class Code>
struct DynQuantG4 {
    static int run(const float* x, int64_t n, void* q, const int2* part, int nparts, float* qp, int qmin, float eps,
                   float width_f, Grid g, hipStream_t st) {
        const dim3 grid = dyn_g4_grid(n);
        auto go = [&](auto u_c) {
            hipLaunchKernelGGL((dyn_quantize_g4_kernel<Code, decltype(u_c)::value>), grid, dim3(kBlock), 0, st, x,
                               (typename Code::T*)q, (uint32_t)n, part, nparts, qp, qmin, eps, width_f, g);
        };
        static_assert(kG4Inflight == 16, "unroll choices");
        switch (dyn_g4_unroll(n, grid.x)) {
        case 1: go(std::integral_constant<int, 1>{}); break;
        case 2: go(std::integral_constant<int, 2>{}); break;
        case 4: go(std::integral_constant<int, 4>{}); break;
        case 8: go(std::integral_constant<int, 8>{}); break;
        default: go(std::integral_constant<int, 16>{}); break;
        }
        return launch_status("lq_dynamic_quantize_f32");
    }
};

// Per-tensor quantize at mid sizes (up to QUANT_AHEAD_MAX values): at most 1024 workgroups,
// each lane's first U groups (the launch's groups per lane rounded up to a power of two) read
// at once, the device scale with them -- one memory round trip where quantize_g4_kernel's
// 4-8192 workgroups of one group per lane queue in waves of resident workgroups.  Same
// arithmetic per group (quantize_group4).
constexpr int64_t QUANT_AHEAD_MAX = (int64_t)1 << 24;

template <class Code, int U>
__global__ __launch_bounds__(kBlock) void quantize_g4_ahead_kernel(const float* __restrict__ x,
                                                                   typename Code::T* __restrict__ q, uint32_t n,
                                                                   QArgs qa, Grid g) {
    typedef Group4<Code> G;
    const BlockRun r = block_run(n >> 2);
    const vf4* x4 = reinterpret_cast<const vf4*>(x);
    const uint32_t last = (n >> 2) - 1;  // n >= 4 on this path
    vf4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t i = r.i + u * kBlock;
        v[u] = __builtin_nontemporal_load(&x4[i < last ? i : last]);
    }
    float t_inv, t_s, t_z;
    qa.tensor(t_inv, t_s, t_z);
    typename G::Raw* q4 = reinterpret_cast<typename G::Raw*>(q);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t i = r.i + u * kBlock;
        if (i < r.end) quantize_group4<Code, PT>(q4, i, v[u], qa, g, t_inv, t_s, t_z);
    }
    quantize_g4_run<Code, PT>(x, q, n, qa, g, t_inv, t_s, t_z, U);
}

template <class Code>
static void launch_quantize_ahead(const float* x, void* q, int64_t n, const QArgs& qa, Grid g, hipStream_t st) {
    const dim3 grid = dyn_g4_grid(n);
    auto go = [&](auto u_c) {
        hipLaunchKernelGGL((quantize_g4_ahead_kernel<Code, decltype(u_c)::value>), grid, dim3(kBlock), 0, st, x,
                           (typename Code::T*)q, (uint32_t)n, qa, g);
    };
    switch (dyn_g4_unroll(n, grid.x)) {
    case 1: go(std::integral_constant<int, 1>{}); break;
    case 2: go(std::integral_constant<int, 2>{}); break;
    case 4: go(std::integral_constant<int, 4>{}); break;
    case 8: go(std::integral_constant<int, 8>{}); break;
    default: go(std::integral_constant<int, 16>{}); break;
    }
}

// The norm before a dynamic Linear at prefill sizes, with the first half of its input step:
// each wave normalizes rows (ln_load / ln_norm, or ln_row_wide past 2048 columns: the bits of
// layer_norm_kernel, x replaced by x + res first when res is given), stores them to y and
// folds the stored values into extrema keys; the workgroup's pair goes to part[blockIdx.x]
// for dyn_quantize_g4_kernel.  At most DYN_PARTS_MAX workgroups, each walking rows
// gridDim.x * 4 apart.
template <int MAXC>
__global__ __launch_bounds__(kBlock) void ln_extrema_kernel(float* x, int64_t ldx, const float* res, int64_t ldres,
                                                            int rows, int D, const float* __restrict__ gamma,
                                                            const float* __restrict__ beta, float ln_eps,
                                                            float* y, int2* __restrict__ part) {
    constexpr int RPW = kBlock / LN_T;  // rows per workgroup pass
    const int wave = threadIdx.x / LN_T, t = threadIdx.x % LN_T;
    int32_t kmin = KEY_POS_INF, kmax = KEY_NEG_INF;
    for (int r = (int)blockIdx.x * RPW + wave; r < rows; r += (int)gridDim.x * RPW) {
        float* xr = x + (int64_t)r * ldx;
        const float* rr = res ? res + (int64_t)r * ldres : nullptr;
        float* yr = y + (int64_t)r * D;
        if constexpr (MAXC == 0) {
            ln_row_wide(xr, rr, true, D, t, gamma, beta, ln_eps, yr);
            for (int c = t; c < (D + 3) >> 2; c += LN_T)  // the lane's own stores, read back
                for (int e = 0; e < 4; ++e)
                    if (4 * c + e < D) key_accum(kmin, kmax, yr[4 * c + e]);
        } else {
            float v[4 * MAXC];
            ln_load<MAXC>(xr, rr, xr, true, D, t, v);
            ln_norm<MAXC>(v, true, D, t, gamma, beta, ln_eps, yr);
#pragma unroll
            for (int j = 0; j < MAXC; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (4 * (t + LN_T * j) + e < D) key_accum(kmin, kmax, v[4 * j + e]);
        }
    }
    block_reduce_keys(kmin, kmax);
    if (threadIdx.x == 0) part[blockIdx.x] = make_int2(kmin, kmax);
}

static int ln_extrema_grid(int64_t rows) {
    const int64_t g = (rows + kBlock / LN_T - 1) / (kBlock / LN_T);
    return (int)(g < DYN_PARTS_MAX ? g : DYN_PARTS_MAX);
}

template <class Code>
struct DynQuantSmall {
    static int run(const float* x, int64_t n, void* q, float* qp, int qmin, float eps, float width_f, Grid g,
                   hipStream_t st) {
        hipLaunchKernelGGL(dyn_quant_small_kernel<Code>, dim3(1), dim3(kDynBlock), 0, st, x, (int)n,
                           (typename Code::T*)q, qp, qmin, eps, width_f, g, aligned16(x));
        return launch_status("lq_dynamic_quantize_f32");
    }
};

// The same step with the input produced in the launch: the layer norm of `rows` rows of D
// (optionally after the residual add x += res, written back), as lq_layer_norm_f32 /
// lq_add_layer_norm_f32 compute it -- one wave per row (ln_load / ln_norm, or ln_row_wide),
// sixteen rows at a time on the workgroup's 1024 threads -- so the codes and qparams are the
// bits of that call followed by lq_dynamic_quantize_f32.  The normalized rows wait in LDS.
// (A GELU before the quantize belongs in the producing GEMM's epilogue instead, LQ_EPI_GELU.)
enum { DQ_LN = 2, DQ_LN_RES = 3 };
constexpr int64_t DQ_LN_MAX = 12288;  // normalized values held in LDS (48 KB)

template <int MAXC>
__device__ __forceinline__ void dq_norm_rows(float* x, int64_t ldx, const float* res, int64_t ldres, int rows,
                                             int D, const float* gamma, const float* beta, float ln_eps, float* ys) {
    const int wave = threadIdx.x / LN_T, t = threadIdx.x % LN_T;
    for (int r = wave; r < rows; r += kDynBlock / LN_T) {
        float* xr = x + (int64_t)r * ldx;
        const float* rr = res ? res + (int64_t)r * ldres : nullptr;
        if constexpr (MAXC == 0) {
            ln_row_wide(xr, rr, true, D, t, gamma, beta, ln_eps, ys + r * D);
        } else {
            float v[4 * MAXC];
            ln_load<MAXC>(xr, rr, xr, true, D, t, v);
            ln_norm<MAXC>(v, true, D, t, gamma, beta, ln_eps, ys + r * D);
        }
    }
}

template <class Code, int SRC>
__global__ __launch_bounds__(kDynBlock) void dyn_quant_fused_kernel(float* x, int64_t ldx, const float* res,
                                                                    int64_t ldres, int rows, int D,
                                                                    const float* __restrict__ gamma,
                                                                    const float* __restrict__ beta, float ln_eps,
                                                                    typename Code::T* __restrict__ q,
                                                                    float* __restrict__ qp, int qmin, float eps,
                                                                    float width_f, Grid g) {
    extern __shared__ float ys[];
    __shared__ int32_t smin[kDynBlock / 64], smax[kDynBlock / 64];
    __shared__ float s_sz[2];
    const int tid = threadIdx.x;
    const int n = rows * D;
    const float* rs = SRC == DQ_LN_RES ? res : nullptr;
    if (D <= 8 * LN_T) dq_norm_rows<2>(x, ldx, rs, ldres, rows, D, gamma, beta, ln_eps, ys);
    else if (D <= 32 * LN_T) dq_norm_rows<8>(x, ldx, rs, ldres, rows, D, gamma, beta, ln_eps, ys);
    else dq_norm_rows<0>(x, ldx, rs, ldres, rows, D, gamma, beta, ln_eps, ys);
    __syncthreads();
    auto val = [&](int i) -> float { return ys[i]; };
    int32_t kmin = KEY_POS_INF, kmax = KEY_NEG_INF;
    for (int i = tid; i < n; i += kDynBlock) key_accum(kmin, kmax, val(i));
    kmin = wave_min(kmin);
    kmax = wave_max(kmax);
    if ((tid & 63) == 0) {
        smin[tid >> 6] = kmin;
        smax[tid >> 6] = kmax;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kDynBlock / 64; ++w) {
            kmin = min(kmin, smin[w]);
            kmax = max(kmax, smax[w]);
        }
        float o[4];
        dyn_qparams(kmin, kmax, qmin, eps, width_f, g, o);
        qp[0] = o[0];
        qp[1] = o[1];
        qp[2] = o[2];
        qp[3] = o[3];
        s_sz[0] = o[2];
        s_sz[1] = o[3];
    }
    __syncthreads();
    const float sc = s_sz[0], z = s_sz[1];
    const float inv = 1.0f / sc;
    for (int i = tid; i < n; i += kDynBlock) q[i] = Code::store(quant_one<Code>(val(i), inv, z, g));
}

template <class Code>
struct DynQuantFused {
    static int run(int src, float* x, int64_t ldx, const float* res, int64_t ldres, int rows, int D,
                   const float* gamma, const float* beta, float ln_eps, void* q, float* qp, int qmin, float eps,
                   float width_f, Grid g, hipStream_t st) {
        typedef typename Code::T T;
        const size_t lds = sizeof(float) * (size_t)rows * D;
#define LQ_DQF(S) \
    hipLaunchKernelGGL((dyn_quant_fused_kernel<Code, S>), dim3(1), dim3(kDynBlock), lds, st, x, ldx, res, ldres, rows, D, \
                       gamma, beta, ln_eps, (T*)q, qp, qmin, eps, width_f, g)
        if (src == DQ_LN) LQ_DQF(DQ_LN);
        else LQ_DQF(DQ_LN_RES);
#undef LQ_DQF
        return launch_status("lq_layer_norm_quantize_f32");
    }
};

template <class Code>
struct QuantPt {
    static int run(const float* x, void* q, int64_t n, PtParams pp, Grid g, hipStream_t st) {
        typedef typename Code::T T;
        if (g4_ok<Code>(x, q, n)) {
            QArgs qa{pp.d_scale, pp.d_zp, pp.inv_value, pp.scale_value, pp.zp_value, 1u, 1u};
            if (n >= 4 && n <= QUANT_AHEAD_MAX)
                launch_quantize_ahead<Code>(x, q, n, qa, g, st);
            else
                hipLaunchKernelGGL((quantize_g4_kernel<Code, PT>), g4_quant_grid(n), dim3(kBlock), 0, st, x, (T*)q,
                                   (uint32_t)n, qa, g);
        } else {
            hipLaunchKernelGGL(quantize_pt_kernel<Code>, scalar_grid(n), dim3(kBlock), 0, st, x, (T*)q, n,
                               pp, g, false);
        }
        return launch_status("lq_quantize_per_tensor_f32");
    }
};

template <class Code>
struct QuantPc {
    static int run(const float* x, void* q, int64_t n, int64_t C, int64_t inner, const float* scale,
                   const float* zp, float zp_value, Grid g, hipStream_t st) {
        typedef typename Code::T T;
        if (g4_ok<Code>(x, q, n)) {
            QArgs qa{scale, zp, 0.f, 0.f, zp_value, (uint32_t)C, (uint32_t)inner};
            if (inner % 4 == 0)
                hipLaunchKernelGGL((quantize_g4_kernel<Code, PCG>), g4_quant_grid(n), dim3(kBlock), 0, st, x,
                                   (T*)q, (uint32_t)n, qa, g);
            else
                hipLaunchKernelGGL((quantize_g4_kernel<Code, PCE>), g4_quant_grid(n), dim3(kBlock), 0, st, x,
                                   (T*)q, (uint32_t)n, qa, g);
        } else {
            hipLaunchKernelGGL(quantize_pc_kernel<Code>, scalar_grid(n), dim3(kBlock), 0, st, x, (T*)q, n,
                               C, inner, scale, zp, zp_value, g, false);
        }
        return launch_status("lq_quantize_per_channel_f32");
    }
};

template <class Code>
struct DequantPt {
    static int run(const void* q, void* y, int y_dtype, int64_t n, PtParams pp, hipStream_t st) {
        typedef typename Code::T T;
        const bool y_ok = (y_dtype == LQ_F32) ? aligned16(y) : (((uintptr_t)y & 7) == 0);
        const uintptr_t ca = 4 * sizeof(T) - 1;
        if (y_ok && ((reinterpret_cast<uintptr_t>(q) & ca) == 0) && n < ((int64_t)1 << 32)) {
            QArgs qa{pp.d_scale, pp.d_zp, pp.inv_value, pp.scale_value, pp.zp_value, 1u, 1u};
            if (y_dtype == LQ_F32)
                hipLaunchKernelGGL((dequantize_g4_kernel<Code, float, PT>), g4_grid(n), dim3(kBlock), 0, st,
                                   (const T*)q, (float*)y, (uint32_t)n, qa);
            else
                hipLaunchKernelGGL((dequantize_g4_kernel<Code, __half, PT>), g4_grid(n), dim3(kBlock), 0,
                                   st, (const T*)q, (__half*)y, (uint32_t)n, qa);
        } else if (y_dtype == LQ_F32) {
            hipLaunchKernelGGL((dequantize_pt_kernel<Code, float>), scalar_grid(n), dim3(kBlock), 0, st,
                               (const T*)q, (float*)y, n, pp, false);
        } else {
            hipLaunchKernelGGL((dequantize_pt_kernel<Code, __half>), scalar_grid(n), dim3(kBlock), 0, st,
                               (const T*)q, (__half*)y, n, pp, false);
        }
        return launch_status("lq_dequantize_per_tensor");
    }
};

template <class Code>
struct DequantPc {
    static int run(const void* q, void* y, int y_dtype, int64_t n, int64_t C, int64_t inner,
                   const float* scale, const float* zp, float zp_value, hipStream_t st) {
        typedef typename Code::T T;
        const bool y_ok = (y_dtype == LQ_F32) ? aligned16(y) : (((uintptr_t)y & 7) == 0);
        const uintptr_t ca = 4 * sizeof(T) - 1;
        if (y_ok && ((reinterpret_cast<uintptr_t>(q) & ca) == 0) && n < ((int64_t)1 << 32)) {
            QArgs qa{scale, zp, 0.f, 0.f, zp_value, (uint32_t)C, (uint32_t)inner};
            const bool grp = inner % 4 == 0;
            if (y_dtype == LQ_F32) {
                if (grp)
                    hipLaunchKernelGGL((dequantize_g4_kernel<Code, float, PCG>), g4_grid(n), dim3(kBlock), 0,
                                       st, (const T*)q, (float*)y, (uint32_t)n, qa);
                else
                    hipLaunchKernelGGL((dequantize_g4_kernel<Code, float, PCE>), g4_grid(n), dim3(kBlock), 0,
                                       st, (const T*)q, (float*)y, (uint32_t)n, qa);
            } else {
                if (grp)
                    hipLaunchKernelGGL((dequantize_g4_kernel<Code, __half, PCG>), g4_grid(n), dim3(kBlock),
                                       0, st, (const T*)q, (__half*)y, (uint32_t)n, qa);
                else
                    hipLaunchKernelGGL((dequantize_g4_kernel<Code, __half, PCE>), g4_grid(n), dim3(kBlock),
                                       0, st, (const T*)q, (__half*)y, (uint32_t)n, qa);
            }
        } else if (y_dtype == LQ_F32) {
            hipLaunchKernelGGL((dequantize_pc_kernel<Code, float>), scalar_grid(n), dim3(kBlock), 0, st,
                               (const T*)q, (float*)y, n, C, inner, scale, zp, zp_value, false);
        } else {
            hipLaunchKernelGGL((dequantize_pc_kernel<Code, __half>), scalar_grid(n), dim3(kBlock), 0, st,
                               (const T*)q, (__half*)y, n, C, inner, scale, zp, zp_value, false);
        }
        return launch_status("lq_dequantize_per_channel");
    }
};

template <int MODE>
static void launch_fq(const float* x, float* y, float* mask, int64_t n, const QArgs& qa, Grid g,
                      hipStream_t st) {
    if (mask)
        hipLaunchKernelGGL((fake_quant_g4_kernel<MODE, true>), g4_grid(n), dim3(kBlock), 0, st, x, y, mask,
                           (uint32_t)n, qa, g);
    else
        hipLaunchKernelGGL((fake_quant_g4_kernel<MODE, false>), g4_grid(n), dim3(kBlock), 0, st, x, y, mask,
                           (uint32_t)n, qa, g);
}

static int check_ocl(int64_t outer, int64_t C, int64_t inner) {
    LQ_REQUIRE(outer >= 0 && C >= 1 && inner >= 0, "invalid [outer, C, inner] layout");
    return LQ_OK;
}

bool dyn_parts_ok(int q_dtype, const void* x, const void* q, int64_t n, int nparts) {
    return n >= 4 && nparts >= 1 && nparts <= DYN_PARTS_MAX && valid_code(q_dtype) && g4_ok_code(q_dtype, x, q, n);
}

int dyn_quantize_parts(const float* x, int64_t n, int q_dtype, int qmin, int qmax, float eps, const int2* parts,
                       int nparts, float* qparams, void* q, hipStream_t st) {
    return dispatch_code<DynQuantG4>(q_dtype, x, n, q, parts, nparts, qparams, qmin, eps, (float)(qmax - qmin),
                                     make_grid(qmin, qmax), st);
}

}  // namespace lq

using namespace lq;

extern "C" {

size_t lq_minmax_workspace_size(int64_t n) { return sizeof(int2) * (size_t)minmax_grid(n); }

int lq_minmax_f32(const float* d_x, int64_t n, float* d_running_min, float* d_running_max,
                  int mode, float ema_c, void* d_workspace, size_t workspace_bytes, void* stream) {
    LQ_REQUIRE(n >= 0, "lq_minmax_f32: n < 0");
    LQ_REQUIRE(d_running_min && d_running_max, "lq_minmax_f32: NULL running buffer");
    LQ_REQUIRE(n == 0 || d_x, "lq_minmax_f32: NULL input");
    LQ_REQUIRE(mode >= 0 && mode <= 2, "lq_minmax_f32: bad mode");
    const int grid = minmax_grid(n);
    LQ_REQUIRE(d_workspace && workspace_bytes >= sizeof(int2) * (size_t)grid,
               "lq_minmax_f32: workspace too small");
    hipStream_t st = as_stream(stream);
    int2* part = (int2*)d_workspace;
    hipLaunchKernelGGL(minmax_partial_kernel, dim3(grid), dim3(kBlock), 0, st, d_x, n, part,
                       aligned16(d_x));
    int rc = launch_status("lq_minmax_f32 partial");
    if (rc) return rc;
    hipLaunchKernelGGL(minmax_finalize_kernel, dim3(1), dim3(kBlock), 0, st, part, grid,
                       d_running_min, d_running_max, mode, ema_c);
    return launch_status("lq_minmax_f32 finalize");
}

size_t lq_minmax_per_channel_workspace_size(int64_t outer, int64_t C, int64_t inner) {
    if (C < 1 || outer < 0 || inner < 0) return 0;
    return pc_plan(outer, C, inner).bytes;
}

int lq_minmax_per_channel_f32(const float* d_x, int64_t outer, int64_t C, int64_t inner,
                              float* d_running_min, float* d_running_max, int mode, float ema_c,
                              void* d_workspace, size_t workspace_bytes, void* stream) {
    int rc = check_ocl(outer, C, inner);
    if (rc) return rc;
    LQ_REQUIRE(d_running_min && d_running_max, "lq_minmax_per_channel_f32: NULL running buffer");
    LQ_REQUIRE(outer * inner == 0 || d_x, "lq_minmax_per_channel_f32: NULL input");
    LQ_REQUIRE(mode >= 0 && mode <= 2, "lq_minmax_per_channel_f32: bad mode");
    PcPlan p = pc_plan(outer, C, inner);
    LQ_REQUIRE(d_workspace && workspace_bytes >= p.bytes,
               "lq_minmax_per_channel_f32: workspace too small");
    LQ_REQUIRE(C <= 0x7fffffff, "lq_minmax_per_channel_f32: too many channels");
    hipStream_t st = as_stream(stream);
    int2* part = (int2*)d_workspace;
    if (p.rows) {
        bool vec = aligned16(d_x) && (inner % 4 == 0);
        hipLaunchKernelGGL(minmax_pc_rows_kernel, dim3((unsigned)C, (unsigned)p.splits), dim3(kBlock),
                           0, st, d_x, outer, C, inner, p.splits, part, vec);
    } else {
        int64_t width = C * inner;
        if (width > 0) {
            int64_t tiles = (width + kBlock - 1) / kBlock;
            LQ_REQUIRE(tiles <= 0x7fffffff, "lq_minmax_per_channel_f32: too wide");
            hipLaunchKernelGGL(minmax_pc_cols_kernel, dim3((unsigned)tiles, (unsigned)p.splits),
                               dim3(kBlock), 0, st, d_x, outer, width, p.splits, part);
        }
    }
    rc = launch_status("lq_minmax_per_channel_f32 partial");
    if (rc) return rc;
    // inner == 0 leaves per_c == 0: the finalize reads no partials and folds the
    // identity extrema {+inf, -inf}.
    hipLaunchKernelGGL(minmax_pc_finalize_kernel, dim3(1), dim3(1024), 0, st, part, p.splits, C,
                       p.per_c, d_running_min, d_running_max, mode, ema_c);
    return launch_status("lq_minmax_per_channel_f32 finalize");
}

int lq_calc_qparams_f32(const float* d_min, const float* d_max, int64_t n, int symmetric,
                        int is_signed, int qmin, int qmax, float eps, float* d_scale,
                        float* d_zero_point, void* stream) {
    LQ_REQUIRE(n >= 0, "lq_calc_qparams_f32: n < 0");
    if (n == 0) return LQ_OK;
    LQ_REQUIRE(d_min && d_max && d_scale && d_zero_point, "lq_calc_qparams_f32: NULL pointer");
    LQ_REQUIRE(qmax > qmin, "lq_calc_qparams_f32: qmax <= qmin");
    // Python-side constants of _qparams.py:197-204, rounded to float32 as the scalars are.
    const float half_range = (float)((double)(qmax - qmin) / 2.0);
    const float width_f = (float)(qmax - qmin);
    // (qmax + qmin + 1) // 2 with Python's floor division.
    const long long sum = (long long)qmax + qmin + 1;
    const long long half = (sum >= 0 || sum % 2 == 0) ? sum / 2 : sum / 2 - 1;
    const float mid_zp = (float)half;
    unsigned blocks = (unsigned)((n + kBlock - 1) / kBlock);
    hipLaunchKernelGGL(calc_qparams_kernel, dim3(blocks), dim3(kBlock), 0, as_stream(stream), d_min,
                       d_max, n, symmetric, is_signed, qmin, qmax, eps, d_scale, d_zero_point,
                       half_range, width_f, mid_zp, make_grid(qmin, qmax));
    return launch_status("lq_calc_qparams_f32");
}

int lq_quantize_per_tensor_f32(const float* d_x, void* d_q, int64_t n, int q_dtype,
                               const float* d_scale, const float* d_zero_point,
                               float inv_scale_value, float zero_point_value, int qmin, int qmax,
                               void* stream) {
    LQ_REQUIRE(n >= 0, "lq_quantize_per_tensor_f32: n < 0");
    if (n == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_q, "lq_quantize_per_tensor_f32: NULL pointer");
    LQ_REQUIRE(valid_code(q_dtype), "lq_quantize_per_tensor_f32: bad code dtype");
    LQ_REQUIRE(qmax >= qmin, "lq_quantize_per_tensor_f32: qmax < qmin");
    PtParams pp{d_scale, d_zero_point, inv_scale_value, 0.0f, zero_point_value};
    return dispatch_code<QuantPt>(q_dtype, d_x, d_q, n, pp, make_grid(qmin, qmax), as_stream(stream));
}

size_t lq_dynamic_quantize_workspace_size(int64_t n) {
    if (n < 0) return 0;
    return (n > 0 && n <= DYN_SMALL_MAX) ? 0 : lq_minmax_workspace_size(n);
}

int lq_dynamic_quantize_f32(const float* d_x, int64_t n, int q_dtype, int qmin, int qmax, float eps, float* d_qparams,
                            void* d_q, void* d_workspace, size_t workspace_bytes, void* stream) {
    LQ_REQUIRE(n >= 0, "lq_dynamic_quantize_f32: n < 0");
    LQ_REQUIRE(d_qparams, "lq_dynamic_quantize_f32: NULL qparams");
    LQ_REQUIRE(n == 0 || (d_x && d_q), "lq_dynamic_quantize_f32: NULL pointer");
    LQ_REQUIRE(valid_code(q_dtype), "lq_dynamic_quantize_f32: bad code dtype");
    LQ_REQUIRE(qmax > qmin, "lq_dynamic_quantize_f32: qmax <= qmin");
    const Grid g = make_grid(qmin, qmax);
    const float width_f = (float)(qmax - qmin);
    hipStream_t st = as_stream(stream);
    if (n > 0 && n <= DYN_SMALL_MAX) {
        note_path("dynamic quantize fused");
        return dispatch_code<DynQuantSmall>(q_dtype, d_x, n, d_q, d_qparams, qmin, eps, width_f, g, st);
    }
    const int parts = minmax_grid(n) < DYN_PARTS_MAX ? minmax_grid(n) : DYN_PARTS_MAX;
    if (n > DYN_SMALL_MAX && g4_ok_code(q_dtype, d_x, d_q, n)) {
        LQ_REQUIRE(d_workspace && workspace_bytes >= sizeof(int2) * (size_t)parts,
                   "lq_dynamic_quantize_f32: workspace too small");
        note_path("dynamic quantize two-launch");
        int2* part = static_cast<int2*>(d_workspace);
        hipLaunchKernelGGL(minmax_partial_kernel, dim3(parts), dim3(kBlock), 0, st, d_x, n, part, true);
        const int rc = launch_status("lq_dynamic_quantize_f32 extrema");
        if (rc) return rc;
        return dispatch_code<DynQuantG4>(q_dtype, d_x, n, d_q, part, parts, d_qparams, qmin, eps, width_f, g, st);
    }
    // the separate launches: observer (replace), qparams, quantize with the device scale
    note_path("dynamic quantize");
    int rc = lq_minmax_f32(d_x, n, d_qparams, d_qparams + 1, LQ_OBS_REPLACE, 0.0f, d_workspace, workspace_bytes,
                           stream);
    if (rc) return rc;
    rc = lq_calc_qparams_f32(d_qparams, d_qparams + 1, 1, 0, 0, qmin, qmax, eps, d_qparams + 2, d_qparams + 3,
                             stream);
    if (rc) return rc;
    return lq_quantize_per_tensor_f32(d_x, d_q, n, q_dtype, d_qparams + 2, d_qparams + 3, 0.0f, 0.0f, qmin, qmax,
                                      stream);
}

int lq_layer_norm_quantize_f32(float* d_x, int64_t ldx, const float* d_res, int64_t ldres, int64_t rows, int64_t D,
                               const float* d_gamma, const float* d_beta, float ln_eps, int q_dtype, int qmin,
                               int qmax, float eps, float* d_qparams, void* d_q, void* stream) {
    LQ_REQUIRE(rows > 0 && D > 0 && ldx >= D && (!d_res || ldres >= D), "lq_layer_norm_quantize_f32: bad shape");
    LQ_REQUIRE(d_x && d_qparams && d_q, "lq_layer_norm_quantize_f32: NULL pointer");
    LQ_REQUIRE(valid_code(q_dtype), "lq_layer_norm_quantize_f32: bad code dtype");
    LQ_REQUIRE(qmax > qmin, "lq_layer_norm_quantize_f32: qmax <= qmin");
    if (rows * D > DQ_LN_MAX)
        return set_error(LQ_ERR_UNSUPPORTED, "lq_layer_norm_quantize_f32: more than 12288 values (one workgroup)");
    return dispatch_code<DynQuantFused>(q_dtype, d_res ? (int)DQ_LN_RES : (int)DQ_LN, d_x, ldx, d_res, ldres,
                                        (int)rows, (int)D, d_gamma, d_beta, ln_eps, d_q, d_qparams, qmin, eps,
                                        (float)(qmax - qmin), make_grid(qmin, qmax), as_stream(stream));
}

size_t lq_layer_norm_dynamic_quantize_workspace_size(int64_t rows, int64_t D) {
    if (rows <= 0 || D <= 0) return 0;
    const size_t ln = sizeof(int2) * (size_t)ln_extrema_grid(rows);
    const size_t dq = lq_dynamic_quantize_workspace_size(rows * D);
    return ln > dq ? ln : dq;
}

int lq_layer_norm_dynamic_quantize_f32(float* d_x, int64_t ldx, const float* d_res, int64_t ldres, int64_t rows,
                                       int64_t D, const float* d_gamma, const float* d_beta, float ln_eps, float* d_y,
                                       int q_dtype, int qmin, int qmax, float eps, float* d_qparams, void* d_q,
                                       void* d_workspace, size_t workspace_bytes, void* stream) {
    const char* fn = "lq_layer_norm_dynamic_quantize_f32";
    LQ_REQUIRE(rows > 0 && D > 0 && D < ((int64_t)1 << 30) && rows <= 0x7fffffff && ldx >= D &&
                   (!d_res || ldres >= D),
               std::string(fn) + ": bad shape");
    LQ_REQUIRE(d_x && d_y && d_qparams && d_q, std::string(fn) + ": NULL pointer");
    LQ_REQUIRE(valid_code(q_dtype), std::string(fn) + ": bad code dtype");
    LQ_REQUIRE(qmax > qmin, std::string(fn) + ": qmax <= qmin");
    LQ_REQUIRE(workspace_bytes >= lq_layer_norm_dynamic_quantize_workspace_size(rows, D) && d_workspace,
               std::string(fn) + ": workspace too small");
    const int64_t n = rows * D;
    hipStream_t st = as_stream(stream);
    if (n > DYN_SMALL_MAX && g4_ok_code(q_dtype, d_y, d_q, n)) {
        note_path("layer norm dynamic quantize two-launch");
        int2* part = static_cast<int2*>(d_workspace);
        const int grid = ln_extrema_grid(rows);
        auto go = [&](auto c) {
            hipLaunchKernelGGL((ln_extrema_kernel<decltype(c)::value>), dim3((unsigned)grid), dim3(kBlock), 0, st, d_x,
                               ldx, d_res, ldres, (int)rows, (int)D, d_gamma, d_beta, ln_eps, d_y, part);
        };
        if (D <= 4 * LN_T) go(std::integral_constant<int, 1>{});
        else if (D <= 8 * LN_T) go(std::integral_constant<int, 2>{});
        else if (D <= 16 * LN_T) go(std::integral_constant<int, 4>{});
        else if (D <= 32 * LN_T) go(std::integral_constant<int, 8>{});
        else go(std::integral_constant<int, 0>{});
        const int rc = launch_status(fn);
        if (rc) return rc;
        return dispatch_code<DynQuantG4>(q_dtype, d_y, n, d_q, part, grid, d_qparams, qmin, (float)eps,
                                         (float)(qmax - qmin), make_grid(qmin, qmax), st);
    }
    // the separate calls
    note_path("layer norm dynamic quantize separate");
    int rc = d_res ? lq_add_layer_norm_f32(d_x, ldx, d_res, ldres, d_y, D, rows, D, d_gamma, d_beta, ln_eps, stream)
                   : lq_layer_norm_f32(d_x, ldx, d_y, D, rows, D, d_gamma, d_beta, ln_eps, stream);
    if (rc) return rc;
    return lq_dynamic_quantize_f32(d_y, n, q_dtype, qmin, qmax, eps, d_qparams, d_q, d_workspace, workspace_bytes,
                                   stream);
}

int lq_quantize_per_channel_f32(const float* d_x, void* d_q, int64_t outer, int64_t C,
                                int64_t inner, int q_dtype, const float* d_scale,
                                const float* d_zero_point, float zero_point_value, int qmin,
                                int qmax, void* stream) {
    int rc = check_ocl(outer, C, inner);
    if (rc) return rc;
    const int64_t n = outer * C * inner;
    if (n == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_q && d_scale, "lq_quantize_per_channel_f32: NULL pointer");
    LQ_REQUIRE(valid_code(q_dtype), "lq_quantize_per_channel_f32: bad code dtype");
    LQ_REQUIRE(qmax >= qmin, "lq_quantize_per_channel_f32: qmax < qmin");
    return dispatch_code<QuantPc>(q_dtype, d_x, d_q, n, C, inner, d_scale, d_zero_point,
                                  zero_point_value, make_grid(qmin, qmax), as_stream(stream));
}

int lq_dequantize_per_tensor(const void* d_q, int q_dtype, void* d_y, int y_dtype, int64_t n,
                             const float* d_scale, const float* d_zero_point, float scale_value,
                             float zero_point_value, void* stream) {
    LQ_REQUIRE(n >= 0, "lq_dequantize_per_tensor: n < 0");
    if (n == 0) return LQ_OK;
    LQ_REQUIRE(d_q && d_y, "lq_dequantize_per_tensor: NULL pointer");
    LQ_REQUIRE(valid_code(q_dtype), "lq_dequantize_per_tensor: bad code dtype");
    LQ_REQUIRE(y_dtype == LQ_F32 || y_dtype == LQ_F16, "lq_dequantize_per_tensor: bad output dtype");
    PtParams pp{d_scale, d_zero_point, 0.0f, scale_value, zero_point_value};
    return dispatch_code<DequantPt>(q_dtype, d_q, d_y, y_dtype, n, pp, as_stream(stream));
}

int lq_dequantize_per_channel(const void* d_q, int q_dtype, void* d_y, int y_dtype, int64_t outer,
                              int64_t C, int64_t inner, const float* d_scale,
                              const float* d_zero_point, float zero_point_value, void* stream) {
    int rc = check_ocl(outer, C, inner);
    if (rc) return rc;
    const int64_t n = outer * C * inner;
    if (n == 0) return LQ_OK;
    LQ_REQUIRE(d_q && d_y && d_scale, "lq_dequantize_per_channel: NULL pointer");
    LQ_REQUIRE(valid_code(q_dtype), "lq_dequantize_per_channel: bad code dtype");
    LQ_REQUIRE(y_dtype == LQ_F32 || y_dtype == LQ_F16, "lq_dequantize_per_channel: bad output dtype");
    return dispatch_code<DequantPc>(q_dtype, d_q, d_y, y_dtype, n, C, inner, d_scale, d_zero_point,
                                    zero_point_value, as_stream(stream));
}

int lq_fake_quantize_per_tensor_f32(const float* d_x, float* d_y, int64_t n, const float* d_scale,
                                    const float* d_zero_point, float inv_scale_value,
                                    float scale_value, float zero_point_value, int qmin, int qmax,
                                    float* d_mask, void* stream) {
    LQ_REQUIRE(n >= 0, "lq_fake_quantize_per_tensor_f32: n < 0");
    if (n == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y, "lq_fake_quantize_per_tensor_f32: NULL pointer");
    LQ_REQUIRE(qmax >= qmin, "lq_fake_quantize_per_tensor_f32: qmax < qmin");
    PtParams pp{d_scale, d_zero_point, inv_scale_value, scale_value, zero_point_value};
    const bool vec = aligned16(d_x) && aligned16(d_y) && (!d_mask || aligned16(d_mask)) && n < ((int64_t)1 << 32);
    if (vec) {
        QArgs qa{d_scale, d_zero_point, inv_scale_value, scale_value, zero_point_value, 1u, 1u};
        launch_fq<PT>(d_x, d_y, d_mask, n, qa, make_grid(qmin, qmax), as_stream(stream));
    } else {
        hipLaunchKernelGGL(fake_quant_kernel, scalar_grid(n), dim3(kBlock), 0, as_stream(stream), d_x, d_y,
                           d_mask, n, (int64_t)1, n, pp, (const float*)nullptr, (const float*)nullptr, 0.0f,
                           make_grid(qmin, qmax), false, false);
    }
    return launch_status("lq_fake_quantize_per_tensor_f32");
}

int lq_fake_quantize_per_channel_f32(const float* d_x, float* d_y, int64_t outer, int64_t C,
                                     int64_t inner, const float* d_scale,
                                     const float* d_zero_point, float zero_point_value, int qmin,
                                     int qmax, float* d_mask, void* stream) {
    int rc = check_ocl(outer, C, inner);
    if (rc) return rc;
    const int64_t n = outer * C * inner;
    if (n == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y && d_scale, "lq_fake_quantize_per_channel_f32: NULL pointer");
    LQ_REQUIRE(qmax >= qmin, "lq_fake_quantize_per_channel_f32: qmax < qmin");
    const bool vec = aligned16(d_x) && aligned16(d_y) && (!d_mask || aligned16(d_mask)) && n < ((int64_t)1 << 32);
    if (vec) {
        QArgs qa{d_scale, d_zero_point, 0.f, 0.f, zero_point_value, (uint32_t)C, (uint32_t)inner};
        if (inner % 4 == 0)
            launch_fq<PCG>(d_x, d_y, d_mask, n, qa, make_grid(qmin, qmax), as_stream(stream));
        else
            launch_fq<PCE>(d_x, d_y, d_mask, n, qa, make_grid(qmin, qmax), as_stream(stream));
    } else {
        PtParams pp{nullptr, nullptr, 0.f, 0.f, 0.f};
        hipLaunchKernelGGL(fake_quant_kernel, scalar_grid(n), dim3(kBlock), 0, as_stream(stream), d_x, d_y,
                           d_mask, n, C, inner, pp, d_scale, d_zero_point, zero_point_value,
                           make_grid(qmin, qmax), true, false);
    }
    return launch_status("lq_fake_quantize_per_channel_f32");
}

}  // extern "C"
