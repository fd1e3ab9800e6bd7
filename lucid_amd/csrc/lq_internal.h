// lq_internal.h -- shared host/device helpers of the gfx950 backend.
//
// Every translation unit is compiled with -ffp-contract=off (see lucid_amd/build.py):
// each float expression below is the IEEE binary32 operation it names, never an FMA,
// so the kernels compute the same bits as Lucid's one-op-per-pass CPU composition.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <string>

#include "lq_api.h"

namespace lq {

// ---------------------------------------------------------------- errors (host)
int set_error(int code, const std::string& msg);
int check_hip(hipError_t e, const char* what);

#define LQ_HIP(call)                                      \
    do {                                                  \
        hipError_t _e = (call);                           \
        if (_e != hipSuccess) return ::lq::check_hip(_e, #call); \
    } while (0)

#define LQ_REQUIRE(cond, msg)                                   \
    do {                                                        \
        if (!(cond)) return ::lq::set_error(LQ_ERR_INVALID, msg); \
    } while (0)

// Records which kernel variant a compute call launched (a static string), readable through
// lq_last_path() on the same thread: tests assert which instantiation a shape reaches.
void note_path(const char* path);

// Compute units of the current device (queried once per device, then cached): the grid
// size of persistent kernels that walk their work items in a loop.
int device_cu_count();

inline int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return check_hip(e, what);
    return LQ_OK;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Native clang vector types (HIP's float4/uint4 are wrapper structs, which the
// nontemporal builtins do not accept).
typedef float vf4 __attribute__((ext_vector_type(4)));
typedef uint32_t vu4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------- device scalar rules

// round half to even (v_rndne_f32): Lucid's lucid.round = vvnintf.
__device__ __forceinline__ float rne(float x) { return __builtin_rintf(x); }

// float -> half, round to nearest even, of an already rounded float32 value.  The empty asm
// hides where the value came from: otherwise the backend may fold fptrunc(fmul(a, b)) into
// v_fma_mix (a * b rounded once, to half), which is not the two roundings the contract
// specifies.
__device__ __forceinline__ __half f32_to_f16_rn(float v) {
    asm volatile("" : "+v"(v));
    return __float2half_rn(v);
}

// float -> bfloat16 bits, round to nearest even on the upper 16 bits (overflow rounds to
// infinity; a NaN stays a quiet NaN of the same sign).
__host__ __device__ inline uint16_t f32_to_bf16_bits(float v) {
    uint32_t u;
    __builtin_memcpy(&u, &v, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__host__ __device__ inline float bf16_bits_to_f32(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float v;
    __builtin_memcpy(&v, &u, 4);
    return v;
}

// A float32 value rounded to the precision of a narrower float type and kept in float32:
// mode 0 none, 1 IEEE half (values past the half range become infinities), 2 bfloat16.
// This is the value of Lucid's astype(x.dtype) of a float32 operand.  round_to is for values
// loaded from memory (no arithmetic to fuse the rounding into, and no barrier that would hold
// back the loads around it); round_result_to for values just computed, whose half rounding
// must not fold into the arithmetic that produced them (see f32_to_f16_rn).
enum { LQ_ROUND_NONE = 0, LQ_ROUND_F16 = 1, LQ_ROUND_BF16 = 2 };
__device__ __forceinline__ float round_to(float v, int mode) {
    // both roundings, then a select: no branch to split the loads around a call site into
    // separately waited groups
    const float h = __half2float(__float2half_rn(v));
    const float b = bf16_bits_to_f32(f32_to_bf16_bits(v));
    return mode == LQ_ROUND_F16 ? h : mode == LQ_ROUND_BF16 ? b : v;
}
__device__ __forceinline__ float round_result_to(float v, int mode) {
    if (mode == LQ_ROUND_F16) return __half2float(f32_to_f16_rn(v));
    return round_to(v, mode);
}

// gelu, tanh form: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) (F.gelu(approximate="tanh")),
// one float32 rounding per operation in this order; shared so a fused kernel gives the same
// bits as the standalone one.
__device__ __forceinline__ float gelu_tanh_f32(float v) {
    const float u = 0.7978845608f * (v + 0.044715f * v * v * v);
    return 0.5f * v * (1.0f + tanhf(u));
}

// Layer norm of one row by a group of LN_T threads (two waves), in one fixed order shared by
// the standalone norm (lq_layer_norm_f32) and the norm fused into a dynamic quantize, so the
// two give the same bits: thread t owns the 4-element chunks c = t, t + LN_T, ... of the row
// (elements 4c .. 4c + 3 below D); the row sum adds each thread's elements in index order,
// then a shuffle tree over each wave, then the two wave sums in order; the variance sums the
// squared deviations the same way.  CACHED keeps the thread's (at most 4 MAXC) values in
// registers between the passes, otherwise they are read again from x.  Every thread of the
// workgroup calls it (it holds barriers); `act` says whether this thread's row exists.  On
// return v[] holds the normalized values of the thread's chunks (CACHED), and the row of x
// holds x + res (res given).  part: 2 floats of LDS per row slot.
constexpr int LN_T = 128;

template <int MAXC, bool CACHED>
__device__ __forceinline__ void ln_row(float* xr, const float* rr, bool act, int D, int t, const float* gamma,
                                       const float* beta, float eps, float (&v)[4 * MAXC], float* part,
                                       float* y) {
    const int lane = t & 63, w = t >> 6;
    const int nch = (D + 3) >> 2;
    auto elem = [&](int j, int e) -> float {  // the current value of chunk j, element e
        if constexpr (CACHED) return v[4 * j + e];
        else return xr[4 * (t + LN_T * j) + e];
    };
    // the residual add, written back (each element by the thread that reads it again)
    if constexpr (CACHED) {
#pragma unroll
        for (int j = 0; j < MAXC; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int idx = 4 * (t + LN_T * j) + e;
                float a = 0.0f;
                if (act && idx < D) {
                    a = xr[idx];
                    if (rr) {
                        a = a + rr[idx];
                        xr[idx] = a;
                    }
                }
                v[4 * j + e] = a;
            }
    } else if (rr && act) {
        for (int c = t; c < nch; c += LN_T)
            for (int e = 0; e < 4; ++e) {
                const int idx = 4 * c + e;
                if (idx < D) xr[idx] = xr[idx] + rr[idx];
            }
    }
    const int jn = CACHED ? MAXC : (nch + LN_T - 1) / LN_T;
    auto row_sum = [&](auto term) -> float {
        float s = 0.0f;
        if (act)
            for (int j = 0; j < jn; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (4 * (t + LN_T * j) + e < D) s += term(elem(j, e));
        for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
        if (lane == 0) part[w] = s;
        __syncthreads();
        const float tot = part[0] + part[1];
        __syncthreads();
        return tot;
    };
    const float mean = row_sum([](float a) { return a; }) / (float)D;
    const float var = row_sum([&](float a) {
                          const float c = a - mean;
                          return c * c;
                      }) / (float)D;
    const float inv = 1.0f / sqrtf(var + eps);
    if (!act) return;
    for (int j = 0; j < jn; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int idx = 4 * (t + LN_T * j) + e;
            if (idx < D) {
                float a = (elem(j, e) - mean) * inv;
                if (gamma) a = a * gamma[idx];
                if (beta) a = a + beta[idx];
                if constexpr (CACHED) v[4 * j + e] = a;
                if (y) y[idx] = a;
            }
        }
}

// clip with NaN pass-through and Lucid's signed-zero tie rule (backend/cpu/Vdsp.cpp:33-62).
__device__ __forceinline__ float clip_tie(float v, float lo, float hi, bool lo_ties, bool hi_ties) {
    if (lo_ties ? v <= lo : v < lo) return lo;
    if (hi_ties ? v >= hi : v > hi) return hi;
    return v;
}

struct Grid {
    float lo, hi;
    bool lo_ties, hi_ties;
    int qlo, qhi;  // the same bounds as integers
};

__host__ __device__ inline Grid make_grid(int qmin, int qmax) {
    Grid g;
    g.lo = (float)qmin;
    g.hi = (float)qmax;
    g.lo_ties = (qmin == 0);  // a +0 floor
    g.hi_ties = false;        // an integer cap is never -0
    g.qlo = qmin;
    g.qhi = qmax;
    return g;
}

__device__ __forceinline__ float clip_grid(float v, const Grid& g) {
    return clip_tie(v, g.lo, g.hi, g.lo_ties, g.hi_ties);
}

// float -> integer storage: saturating, NaN -> 0 (backend/cpu/methods/Factory.cpp:127-146).
template <typename T>
__device__ __forceinline__ T satcast(float v, float lo, float hi, int lo_i, int hi_i) {
    if (v != v) return (T)0;
    if (v <= lo) return (T)lo_i;
    if (v >= hi) return (T)hi_i;
    return (T)(int)v;
}

// Code storage types.  store(c) writes the clipped float code c.
struct CodeI8 {
    typedef int8_t T;
    static constexpr int kLo = -128, kHi = 127;
    static __device__ __forceinline__ T from_int(int c) { return (T)c; }
    static __device__ __forceinline__ T store(float c) { return satcast<int8_t>(c, -128.f, 127.f, -128, 127); }
    static __device__ __forceinline__ float load(T v) { return (float)v; }
};
struct CodeU8 {
    typedef uint8_t T;
    static constexpr int kLo = 0, kHi = 255;
    static __device__ __forceinline__ T from_int(int c) { return (T)c; }
    static __device__ __forceinline__ T store(float c) { return satcast<uint8_t>(c, 0.f, 255.f, 0, 255); }
    static __device__ __forceinline__ float load(T v) { return (float)v; }
};
struct CodeI16 {
    typedef int16_t T;
    static constexpr int kLo = -32768, kHi = 32767;
    static __device__ __forceinline__ T from_int(int c) { return (T)c; }
    static __device__ __forceinline__ T store(float c) {
        return satcast<int16_t>(c, -32768.f, 32767.f, -32768, 32767);
    }
    static __device__ __forceinline__ float load(T v) { return (float)v; }
};
struct CodeI32 {
    typedef int32_t T;
    static constexpr int kLo = INT32_MIN, kHi = INT32_MAX;
    static __device__ __forceinline__ T from_int(int c) { return (T)c; }
    static __device__ __forceinline__ T store(float c) {
        if (c != c) return 0;
        if (c <= -2147483648.f) return INT32_MIN;
        if (c >= 2147483648.f) return INT32_MAX;
        return (int32_t)c;
    }
    static __device__ __forceinline__ float load(T v) { return (float)v; }
};
// Unsigned-grid code c kept as int8 (c - 128): the signed MFMA operand form.
struct CodeU8S8 {
    typedef int8_t T;
    static constexpr int kLo = 0, kHi = 255;
    static __device__ __forceinline__ T from_int(int c) { return (T)(c - 128); }
    static __device__ __forceinline__ T store(float c) {
        return (int8_t)((int)satcast<uint8_t>(c, 0.f, 255.f, 0, 255) - 128);
    }
    static __device__ __forceinline__ float load(T v) { return (float)((int)v + 128); }
};

// Saturating float -> int32 conversion (v_cvt_i32_f32: truncates toward zero, out-of-range
// values clamp to the int32 range, NaN converts to 0).
__device__ __forceinline__ int32_t cvt_i32_sat(float v) {
    int32_t r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// Stored code of x quantized onto grid g: Code::store(clip_grid(rne(x * inv) + z, g)),
// computed in the integer domain.  The two agree for every input: the signed-zero tie rule
// of clip_grid cannot change an integer code, truncating then clamping to integer bounds
// equals clamping then truncating, infinities and out-of-range values saturate in both, and
// NaN stores 0 in both (the nan_fix select restores 0 when the grid excludes it).
template <class Code>
__device__ __forceinline__ typename Code::T quant_store(float x, float inv, float z, const Grid& g) {
    const float u = rne(x * inv) + z;
    const int lo = min(max(g.qlo, Code::kLo), Code::kHi);
    const int hi = max(min(g.qhi, Code::kHi), Code::kLo);
    int c = min(max(cvt_i32_sat(u), lo), hi);
    if (!(lo <= 0 && 0 <= hi) && u != u) c = 0;
    return Code::from_int(c);
}

// Order-preserving int32 key of a float: integer order of keys is the float order with
// -0 below +0; a NaN with the sign bit clear keys above +inf, one with it set below -inf.
__device__ __forceinline__ int32_t fkey(float f) {
    int32_t b = __float_as_int(f);
    return b ^ ((b >> 31) & 0x7fffffff);
}
__device__ __forceinline__ float unkey(int32_t k) {
    return __int_as_float(k ^ ((k >> 31) & 0x7fffffff));
}
constexpr int32_t KEY_POS_INF = 0x7f800000;
constexpr int32_t KEY_NEG_INF = (int32_t)(0xff800000u ^ 0x7fffffffu);

// NaN-propagating extreme with -0 < +0 (backend/cpu/Reduce.cpp:54-72).
__device__ __forceinline__ float extreme_min(float a, float b) {
    if (a != a || b != b) return __int_as_float(0x7fc00000);
    return unkey(min(fkey(a), fkey(b)));
}
__device__ __forceinline__ float extreme_max(float a, float b) {
    if (a != a || b != b) return __int_as_float(0x7fc00000);
    return unkey(max(fkey(a), fkey(b)));
}

// Wave64 reductions over int32.
__device__ __forceinline__ int32_t wave_min(int32_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = min(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ int32_t wave_max(int32_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
    return v;
}

}  // namespace lq
