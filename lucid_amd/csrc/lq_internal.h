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

// gelu, tanh form: 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3) (F.gelu(approximate=
// "tanh")), evaluated as x / (1 + e^{-2u}) -- the same function (1 + tanh u = 2 / (1 + e^{-2u}))
// without the cancellation of 1 + tanh u where tanh u is near -1 -- with the hardware exp2 and
// reciprocal (a few ulps; tanhf's libm call was most of a GELU epilogue's VALU work).  Shared
// so a fused kernel gives the same bits as the standalone one.
__device__ __forceinline__ float gelu_tanh_f32(float v) {
    const float u = 0.7978845608f * (v + 0.044715f * v * v * v);
    const float e = __builtin_amdgcn_exp2f(-2.8853900817779268f * u);  // e^{-2u} = 2^{-2u log2 e}
    return v * __builtin_amdgcn_rcpf(1.0f + e);
}

// Layer norm of one row by one wave (LN_T lanes), in one fixed order shared by every kernel
// that normalizes -- the standalone lq_layer_norm_f32 / lq_add_layer_norm_f32, the norm fused
// into a dynamic quantize, the norm folded into a one-launch dynamic Linear -- so all give the
// same bits: lane t owns the 4-element chunks c = t, t + LN_T, ... of the row (elements
// 4c .. 4c + 3 below D); the row sum adds a lane's elements in index order, then a shuffle
// tree over the wave; the variance sums the squared deviations the same way;
// inv = 1 / sqrt(var + eps) and y = ((v - mean) inv) gamma + beta.  A wave owns its row: no
// barrier, so rows in flight are limited only by registers.
constexpr int LN_T = 64;

// The values of a row into v (MAXC chunks per lane) and, with res, its residual terms into rv;
// positions past D, and every position of a row that is not `act`, hold 0.  Loads only, so a
// caller can have several rows in flight before ln_add_store.
template <int MAXC>
__device__ __forceinline__ void ln_fetch(const float* xr, const float* rr, bool act, int D, int t,
                                         float (&v)[4 * MAXC], float (&rv)[4 * MAXC]) {
    // whole 16-byte chunks when D % 4 == 0 and the rows are 16-byte aligned
    const bool vec = (D & 3) == 0 && ((reinterpret_cast<uintptr_t>(xr) | reinterpret_cast<uintptr_t>(rr)) & 15) == 0;
    if (vec) {
#pragma unroll
        for (int j = 0; j < MAXC; ++j) {
            const int idx = 4 * (t + LN_T * j);
            const bool in = act && idx < D;
            const vf4 a = in ? *reinterpret_cast<const vf4*>(xr + idx) : vf4{0.0f, 0.0f, 0.0f, 0.0f};
            const vf4 b = (in && rr) ? *reinterpret_cast<const vf4*>(rr + idx) : vf4{0.0f, 0.0f, 0.0f, 0.0f};
            v[4 * j] = a.x, v[4 * j + 1] = a.y, v[4 * j + 2] = a.z, v[4 * j + 3] = a.w;
            rv[4 * j] = b.x, rv[4 * j + 1] = b.y, rv[4 * j + 2] = b.z, rv[4 * j + 3] = b.w;
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < MAXC; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int idx = 4 * (t + LN_T * j) + e;
            const bool in = act && idx < D;
            v[4 * j + e] = in ? xr[idx] : 0.0f;
            rv[4 * j + e] = (in && rr) ? rr[idx] : 0.0f;
        }
}

// The row's values from v to dst (positions below D): one 16-byte store per chunk when D % 4
// == 0 and dst is 16-byte aligned, else element by element.
template <int MAXC>
__device__ __forceinline__ void ln_store(float* dst, const float (&v)[4 * MAXC], int D, int t) {
    if ((D & 3) == 0 && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
#pragma unroll
        for (int j = 0; j < MAXC; ++j) {
            const int idx = 4 * (t + LN_T * j);
            if (idx < D)
                *reinterpret_cast<vf4*>(dst + idx) = vf4{v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]};
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < MAXC; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int idx = 4 * (t + LN_T * j) + e;
            if (idx < D) dst[idx] = v[4 * j + e];
        }
}

// v = x + res (has_res), stored to wb when it is not NULL (the row of x itself for the in-place
// callers: every load of the row came first).
template <int MAXC>
__device__ __forceinline__ void ln_add_store(float (&v)[4 * MAXC], const float (&rv)[4 * MAXC], bool has_res,
                                             float* wb, bool act, int D, int t) {
    if (!has_res) return;
#pragma unroll
    for (int k = 0; k < 4 * MAXC; ++k) v[k] = v[k] + rv[k];
    if (wb && act) ln_store<MAXC>(wb, v, D, t);
}

template <int MAXC>
__device__ __forceinline__ void ln_load(const float* xr, const float* rr, float* wb, bool act, int D, int t,
                                        float (&v)[4 * MAXC]) {
    float rv[4 * MAXC];
    ln_fetch<MAXC>(xr, rr, act, D, t, v, rv);
    ln_add_store<MAXC>(v, rv, rr != nullptr, wb, act, D, t);
}

// Sum over the 64 lanes of a wave, the same value in every lane: partners at lane distance 1
// and 2 (quad permutes), then the mirrored lane of each 8 and of each 16 (DPP row mirrors),
// then the lane 16 and 32 away (permlane swaps) -- each step adds two partial sums that every
// lane of the pair holds, so all lanes add the same values in the same order.  Register
// permutes only: no LDS round trip per step.
__device__ __forceinline__ float dpp_add(float s, int ctrl_sel) {
    int b = __float_as_int(s), o;
    switch (ctrl_sel) {  // the DPP control must be a constant
    case 0: o = __builtin_amdgcn_update_dpp(b, b, 0xB1, 0xF, 0xF, true); break;   // quad_perm [1,0,3,2]
    case 1: o = __builtin_amdgcn_update_dpp(b, b, 0x4E, 0xF, 0xF, true); break;   // quad_perm [2,3,0,1]
    case 2: o = __builtin_amdgcn_update_dpp(b, b, 0x141, 0xF, 0xF, true); break;  // row_half_mirror
    default: o = __builtin_amdgcn_update_dpp(b, b, 0x140, 0xF, 0xF, true); break; // row_mirror
    }
    return s + __int_as_float(o);
}
__device__ __forceinline__ float ln_wave_sum(float s) {
    s = dpp_add(s, 0);
    s = dpp_add(s, 1);
    s = dpp_add(s, 2);
    s = dpp_add(s, 3);
    const int lane = __lane_id();
    const uint32_t b = __float_as_uint(s);
    auto p16 = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    s = s + __uint_as_float(((lane >> 4) & 1) ? p16[0] : p16[1]);
    const uint32_t c = __float_as_uint(s);
    auto p32 = __builtin_amdgcn_permlane32_swap(c, c, false, false);
    s = s + __uint_as_float(lane >= 32 ? p32[0] : p32[1]);
    return s;
}

// Normalizes the values ln_load left in v, in place, and stores them to y (when not NULL and
// the row is `act`).  Every lane of the wave calls it (the sums are shuffles).
template <int MAXC>
__device__ __forceinline__ void ln_norm(float (&v)[4 * MAXC], bool act, int D, int t, const float* gamma,
                                        const float* beta, float eps, float* y) {
    float gv[4 * MAXC], bv[4 * MAXC];  // the affine terms, loaded under the reductions
#pragma unroll
    for (int j = 0; j < MAXC; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int idx = 4 * (t + LN_T * j) + e;
            const bool in = act && idx < D;
            gv[4 * j + e] = (in && gamma) ? gamma[idx] : 1.0f;
            bv[4 * j + e] = (in && beta) ? beta[idx] : 0.0f;
        }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < MAXC; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (4 * (t + LN_T * j) + e < D) s += v[4 * j + e];
    const float mean = ln_wave_sum(s) / (float)D;
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < MAXC; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (4 * (t + LN_T * j) + e < D) {
                const float c = v[4 * j + e] - mean;
                q += c * c;
            }
    const float var = ln_wave_sum(q) / (float)D;
    const float inv = 1.0f / sqrtf(var + eps);
    if (!act) return;
#pragma unroll
    for (int j = 0; j < MAXC; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int idx = 4 * (t + LN_T * j) + e;
            if (idx < D) {
                float a = (v[4 * j + e] - mean) * inv;
                if (gamma) a = a * gv[4 * j + e];
                if (beta) a = a + bv[4 * j + e];
                v[4 * j + e] = a;
            }
        }
    if (y) ln_store<MAXC>(y, v, D, t);
}

// A row too wide for registers: the same order, read from memory on each pass; x + res is
// stored into the row itself first (in place).
__device__ __forceinline__ void ln_row_wide(float* xr, const float* rr, bool act, int D, int t, const float* gamma,
                                            const float* beta, float eps, float* y) {
    const int nch = (D + 3) >> 2;
    if (rr && act)
        for (int c = t; c < nch; c += LN_T)
            for (int e = 0; e < 4; ++e) {
                const int idx = 4 * c + e;
                if (idx < D) xr[idx] = xr[idx] + rr[idx];
            }
    float s = 0.0f;
    if (act)
        for (int c = t; c < nch; c += LN_T)
            for (int e = 0; e < 4; ++e)
                if (4 * c + e < D) s += xr[4 * c + e];
    const float mean = ln_wave_sum(s) / (float)D;
    float q = 0.0f;
    if (act)
        for (int c = t; c < nch; c += LN_T)
            for (int e = 0; e < 4; ++e)
                if (4 * c + e < D) {
                    const float d = xr[4 * c + e] - mean;
                    q += d * d;
                }
    const float var = ln_wave_sum(q) / (float)D;
    const float inv = 1.0f / sqrtf(var + eps);
    if (!act) return;
    for (int c = t; c < nch; c += LN_T)
        for (int e = 0; e < 4; ++e) {
            const int idx = 4 * c + e;
            if (idx < D) {
                float a = (xr[idx] - mean) * inv;
                if (gamma) a = a * gamma[idx];
                if (beta) a = a + beta[idx];
                y[idx] = a;
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

__device__ __forceinline__ void key_accum(int32_t& kmin, int32_t& kmax, float v) {
    int32_t k = fkey(v);
    kmin = min(kmin, k);
    kmax = max(kmax, k);
}

// Extrema back from their keys; NaN for both when a NaN was seen (a key outside the range
// of ordered floats).
__device__ __forceinline__ void decode_keys(int32_t kmin, int32_t kmax, float& mn, float& mx) {
    if (kmax > KEY_POS_INF || kmin < KEY_NEG_INF) {
        mn = mx = __int_as_float(0x7fc00000);
    } else {
        mn = unkey(kmin);
        mx = unkey(kmax);
    }
}

// Code of x on grid g as a float: clip(rne(x * inv) + z) (the quantize formula).
template <class Code>
__device__ __forceinline__ float quant_one(float x, float inv, float z, const Grid& g) {
    float t = x * inv;
    float r = rne(t);
    float u = r + z;
    return clip_grid(u, g);
}

// Per-tensor affine qparams of a dynamic input from the keys of its extrema (the observer's
// min / max, then calculate_qparams on the grid of width width_f = qmax - qmin):
// out = {min, max, scale, zero point}.
__device__ __forceinline__ void dyn_qparams(int32_t kmin, int32_t kmax, int qmin, float eps, float width_f,
                                            const Grid& g, float (&out)[4]) {
    float cmin, cmax;
    decode_keys(kmin, kmax, cmin, cmax);
    const float mn = extreme_min(cmin, 0.0f), mx = extreme_max(cmax, 0.0f);
    const float wd = mx - mn;
    const float qq = wd / width_f;
    const float sc = extreme_max(qq, eps);
    const float r = rne(mn / sc);
    out[0] = cmin;
    out[1] = cmax;
    out[2] = sc;
    out[3] = clip_grid((float)qmin - r, g);
}

// The second launch of a dynamic quantize whose extrema were folded by the producing kernel:
// nparts (<= DYN_PARTS_MAX) key pairs [min, max] per workgroup of the producer, then every
// workgroup folds them, derives the per-tensor qparams of lq_dynamic_quantize_f32 and
// quantizes x[n] (lq_quant.hip).  dyn_parts_ok: at least one group of four values, x and q
// aligned for the four-code groups, n within 32 bits; otherwise the caller runs
// lq_dynamic_quantize_f32 itself.
constexpr int DYN_PARTS_MAX = 1024;
bool dyn_parts_ok(int q_dtype, const void* x, const void* q, int64_t n, int nparts);
int dyn_quantize_parts(const float* x, int64_t n, int q_dtype, int qmin, int qmax, float eps, const int2* parts,
                       int nparts, float* qparams, void* q, hipStream_t st);

// Wave64 reductions over int32.
// The same pairings as ln_wave_sum (quad permutes, row half-mirror and mirror, then the
// permlane swaps of 16 and 32), with min / max in place of the add: register permutes only,
// where a shuffle ladder waits on six LDS-crossbar round trips.  Min and max are order-free,
// so every lane ends with the wave's extremum.
template <bool MIN>
__device__ __forceinline__ int32_t wave_extreme(int32_t v) {
    auto pick = [](int32_t a, int32_t b) { return MIN ? min(a, b) : max(a, b); };
    v = pick(v, __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, true));   // quad_perm [1,0,3,2]
    v = pick(v, __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, true));   // quad_perm [2,3,0,1]
    v = pick(v, __builtin_amdgcn_update_dpp(v, v, 0x141, 0xF, 0xF, true));  // row_half_mirror
    v = pick(v, __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, true));  // row_mirror
    const int lane = __lane_id();
    const auto p16 = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
    v = pick(v, (int32_t)(((lane >> 4) & 1) ? p16[0] : p16[1]));
    const auto p32 = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    v = pick(v, (int32_t)(lane >= 32 ? p32[0] : p32[1]));
    return v;
}
__device__ __forceinline__ int32_t wave_min(int32_t v) { return wave_extreme<true>(v); }
__device__ __forceinline__ int32_t wave_max(int32_t v) { return wave_extreme<false>(v); }

}  // namespace lq
