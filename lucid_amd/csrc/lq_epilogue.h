// lq_epilogue.h -- the fused W8A8 epilogue shared by the GEMM and the implicit-GEMM conv.
//
// From an exact int32 accumulator (zero points already corrected):
//   y = fl32(fl32(float(acc) * fl32(sa * sb)) + bias), ReLU (y <= 0 -> +0), then the output
//   kind: int32 / f32 / f16 / requantized codes c = clip(rne(y * fl32(1/S)) + Z) of an int8,
//   uint8, int16 or uint8-as-int8 grid / fake-quantized f32 fl32((c - Z) * S).
// Every float op is one IEEE binary32 operation (the translation units build with
// -ffp-contract=off).
#pragma once

#include <hip/hip_fp16.h>

#include <utility>

#include "lq_internal.h"

namespace lq {

struct EpiParams {
    int za;       // effective activation zero point in A's stored units
    bool has_za;
    float out_inv, out_s, out_z;
    Grid g;
};

__device__ __forceinline__ float requant_code(float y, const EpiParams& p) {
    float t = y * p.out_inv;
    float r = rne(t);
    float u = r + p.out_z;
    return clip_grid(u, p.g);
}

// Epilogue value of one element, as the bits of the output element type.
// gelu (float32 output only): the tanh GELU of y after the bias, the float module that follows
// the Linear (gelu_tanh_f32, the bits of the standalone kernel).
template <int KIND>
__device__ __forceinline__ uint32_t epi_one(int32_t acc, float sa, float sb, const float* bias_p,
                                            bool relu, const EpiParams& p, bool gelu = false) {
    if (KIND == LQ_OUT_I32) return (uint32_t)acc;
    float s = sa * sb;
    float y = (float)acc * s;
    if (bias_p) y = y + *bias_p;  // no add without a bias: -0 stays -0
    if (relu) y = (y <= 0.0f) ? 0.0f : y;
    if (KIND == LQ_OUT_F32) return __float_as_uint(gelu ? gelu_tanh_f32(y) : y);
    if (KIND == LQ_OUT_F16) return (uint32_t)__half_as_ushort(f32_to_f16_rn(y));
    float c = requant_code(y, p);
    if (KIND == LQ_OUT_Q8) return (uint32_t)(uint8_t)CodeI8::store(c);
    if (KIND == LQ_OUT_QU8) return (uint32_t)CodeU8::store(c);
    if (KIND == LQ_OUT_Q16) return (uint32_t)(uint16_t)CodeI16::store(c);
    if (KIND == LQ_OUT_QU8S8) return (uint32_t)(uint8_t)CodeU8S8::store(c);
    // LQ_OUT_FQ32
    float d = c - p.out_z;
    return __float_as_uint(d * p.out_s);
}

// Requantized codes of the integer output kinds, clamped first to the grid [qmin, qmax] and
// then to the storage range; lo / hi fold the two clamps into one.  NaN becomes code 0 (the
// saturating cast of Lucid's Factory.cpp:127-146) whatever the grid: cvt_i32_sat gives 0,
// and nan_fix restores 0 when the clamp would move it.
struct CodeClamp {
    int lo, hi;
    bool nan_fix;
};

template <int KIND>
__device__ __forceinline__ CodeClamp code_clamp(int qmin, int qmax) {
    int slo = -128, shi = 127;
    if (KIND == LQ_OUT_QU8 || KIND == LQ_OUT_QU8S8) slo = 0, shi = 255;
    if (KIND == LQ_OUT_Q16) slo = -32768, shi = 32767;
    CodeClamp c;
    c.lo = min(max(qmin, slo), shi);
    c.hi = max(min(qmax, shi), slo);
    c.nan_fix = !(c.lo <= 0 && 0 <= c.hi);
    return c;
}

template <int KIND>
__device__ __forceinline__ int32_t requant_int(float y, const EpiParams& p, const CodeClamp& cc) {
    const float t = y * p.out_inv;
    const float r = rne(t);
    const float u = r + p.out_z;
    int32_t c = min(max(cvt_i32_sat(u), cc.lo), cc.hi);
    if (cc.nan_fix && u != u) c = 0;
    return c;
}

template <int KIND>
struct OutTraits {
    static constexpr int bytes = (KIND == LQ_OUT_I32 || KIND == LQ_OUT_F32 || KIND == LQ_OUT_FQ32) ? 4
                                 : (KIND == LQ_OUT_F16 || KIND == LQ_OUT_Q16)                        ? 2
                                                                                                     : 1;
};

template <int KIND>
__device__ __forceinline__ void store_elem(void* C, int64_t idx, uint32_t v) {
    constexpr int b = OutTraits<KIND>::bytes;
    if (b == 4) reinterpret_cast<uint32_t*>(C)[idx] = v;
    else if (b == 2) reinterpret_cast<uint16_t*>(C)[idx] = (uint16_t)v;
    else reinterpret_cast<uint8_t*>(C)[idx] = (uint8_t)v;
}

// v_med3_i32: the median of x, lo, hi, which is min(max(x, lo), hi) whenever lo <= hi (one
// instruction where the compiler, not knowing lo <= hi, emits two).
__device__ __forceinline__ int32_t med3_i32(int32_t x, int32_t lo, int32_t hi) {
    int32_t r;
    asm("v_med3_i32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(lo), "v"(hi));
    return r;
}

// Round-to-nearest-even of t to an integer, carried in the bit pattern of a float:
// t + 1.5 * 2^23 lies in [2^23, 2^24) for |t| < 2^22, where binary32 spacing is exactly 1, so
// the one IEEE addition rounds t to an integer with ties to even (1.5 * 2^23 is even) and the
// bits are RNE_MAGIC_BITS + rne(t).  Outside that range the bits stay ordered for a clamp to
// [lo, hi] + RNE_MAGIC_BITS with |lo|, |hi| < 2^22: t >= 2^22 gives bits >= 0x4B800000, t <=
// -2^22 gives bits <= 0x4B000000 or a negative int (t + magic < 0, or -inf), +inf 0x7F800000.
// NaN is not ordered (its bits read as the largest positive values): callers exclude it.
// RNE_MAGIC_BITS has zero low 16 bits, so after the clamp the low byte / halfword of the bits
// is the code itself: no conversion back to an integer is needed for 8- and 16-bit stores.
constexpr int32_t RNE_MAGIC_BITS = 0x4B400000;
__device__ __forceinline__ int32_t rne_bits(float t) { return __float_as_int(t + 12582912.0f); }

// The low bytes of v[0..3] as one dword (byte d = v[d] & 0xff): three v_perm_b32.
__device__ __forceinline__ uint32_t pack_low_bytes(const uint32_t* v) {
    // v_perm_b32 selects bytes of {src0, src1} (src1 = bytes 0-3, src0 = 4-7; 0x0c gives 0)
    const uint32_t lo = __builtin_amdgcn_perm(v[1], v[0], 0x0c0c0400u);  // v0.b0, v1.b0, 0, 0
    const uint32_t hi = __builtin_amdgcn_perm(v[3], v[2], 0x0c0c0400u);  // v2.b0, v3.b0, 0, 0
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);                    // lo.b0, lo.b1, hi.b0, hi.b1
}

// Calls f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>): a loop whose body
// indexes register arrays, unrolled whatever the body's size (a loop the unroller leaves
// rolled turns such an array into scratch memory).
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    [&]<int... Is>(std::integer_sequence<int, Is...>) {
        (f(std::integral_constant<int, Is>()), ...);
    }(std::make_integer_sequence<int, N>());
}

}  // namespace lq
