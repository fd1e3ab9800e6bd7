// lq_act.hip -- the float and the quantized activations of a quantized region.
//
// Lucid's quantized activations (lucid/nn/quantized/activation.py:20-475) are the float
// activation followed by a fake-quantize onto a calibrated grid; the float modules
// (nn.Sigmoid, nn.Tanh, nn.Hardswish, nn.Hardsigmoid, nn.ELU, nn.LeakyReLU) run the same
// activation during calibration.  One kernel covers both: it reads float32 or the integer
// codes of a code-backed activation (dequantized as fl32(fl32(float(c) - z) * s), as
// lucid/quantization/_functional.py:293), applies the activation with the operation order of
// Lucid's CPU kernels, and stores float32 or the codes on the output grid
// (clip(rne(t * fl32(1 / S)) + Z), integer domain, NaN -> 0).
//
// Per element (lucid/_C/backend/cpu/methods/Activation.cpp):
//   sigmoid      1 / (1 + exp(-x))                        (:8-50: negate, exp, add, reciprocal)
//   tanh         tanh(x)                                  (Unary.cpp:165-170)
//   hardsigmoid  min(max((x + 3) / 6, 0), 1)               (:661-686; std::max / std::min,
//                                                            so NaN and -0 pass)
//   hardswish    x * hardsigmoid(x)                       (:726-751)
//   elu          x >= 0 ? x : alpha * (exp(x) - 1)        (:435-460)
//   leaky_relu   x >= 0 ? x : slope * x                   (:375-400)
// Division is IEEE (correctly rounded); exp / tanh are the device library's (within an ulp of
// the reference's vForce results, which are not specified to the bit).
//
// Work split: each thread owns groups of E consecutive elements, E = 16 bytes over the wider
// of the input and output element sizes, so every load and store is one 4-16 byte access,
// with eight groups in flight; workgroups take contiguous runs of groups.  Misaligned pointers
// fall back to one element per step.  One-byte code inputs read a 256-entry table of outputs
// built per workgroup in LDS instead of evaluating the activation per element.
#include <hip/hip_runtime.h>

#include <float.h>

#include <type_traits>

#include "lq_internal.h"

namespace lq {

constexpr int kActBlock = 256;

template <int T>
struct ElemOf;
template <> struct ElemOf<LQ_F32> { using type = float; };
template <> struct ElemOf<LQ_I8> { using type = int8_t; };
template <> struct ElemOf<LQ_U8> { using type = uint8_t; };
template <> struct ElemOf<LQ_I16> { using type = int16_t; };
template <> struct ElemOf<LQ_U8S8> { using type = int8_t; };

template <int BYTES>
struct RawVec;
template <> struct RawVec<1> { using type = uint8_t; };
template <> struct RawVec<2> { using type = uint16_t; };
template <> struct RawVec<4> { using type = uint32_t; };
template <> struct RawVec<8> { typedef uint32_t type __attribute__((ext_vector_type(2))); };
template <> struct RawVec<16> { using type = vu4; };

struct ActArgs {
    int op;
    const void* x;
    const float* x_scale;
    const float* x_zp;
    int64_t n;
    float param;
    const float* out_scale;
    const float* out_zp;
    Grid g;
    void* y;
    int vec;
};

template <int IN>
__device__ __forceinline__ float act_in(typename ElemOf<IN>::type v, float s, float z) {
    if constexpr (IN == LQ_F32) {
        return v;
    } else {
        const float c = (IN == LQ_U8S8) ? (float)((int)v + 128) : (float)v;
        const float d = c - z;
        return d * s;
    }
}

// fl32(t / 6): a multiply by fl32(1/6) and one fma residual step, which gives the IEEE
// quotient for every float32 with 2^-125 <= |t| <= FLT_MAX (checked exhaustively over all 2^32
// inputs by the oracle's lqo_div6_mismatches); the IEEE division elsewhere.
__device__ __forceinline__ float div6(float t) {
    constexpr float r = 1.0f / 6.0f;
    const float a = fabsf(t);
    if (a >= 0x1p-125f && a <= FLT_MAX) {
        const float q0 = t * r;
        const float e = __builtin_fmaf(-q0, 6.0f, t);
        return __builtin_fmaf(e, r, q0);
    }
    return t / 6.0f;
}

// std::max(t, 0) then std::min(t, 1): a NaN or a -0 passes both.
__device__ __forceinline__ float hard_sigmoid(float x) {
    float t = div6(x + 3.0f);
    t = (t < 0.0f) ? 0.0f : t;
    t = (1.0f < t) ? 1.0f : t;
    return t;
}

__device__ __forceinline__ float act_apply(int op, float x, float p) {
    switch (op) {
        case LQ_ACT_SIGMOID: {
            const float e = expf(-x);
            const float d = 1.0f + e;
            return 1.0f / d;
        }
        case LQ_ACT_TANH:
            return tanhf(x);
        case LQ_ACT_HARDSWISH:
            return x * hard_sigmoid(x);
        case LQ_ACT_HARDSIGMOID:
            return hard_sigmoid(x);
        case LQ_ACT_ELU: {
            const float em1 = expf(x) - 1.0f;
            return x >= 0.0f ? x : p * em1;
        }
        default:  // LQ_ACT_LEAKY_RELU
            return x >= 0.0f ? x : p * x;
    }
}

template <int OUT>
__device__ __forceinline__ typename ElemOf<OUT>::type act_out(float t, float inv, float z, const Grid& g) {
    if constexpr (OUT == LQ_F32) return t;
    else if constexpr (OUT == LQ_I8) return quant_store<CodeI8>(t, inv, z, g);
    else if constexpr (OUT == LQ_U8) return quant_store<CodeU8>(t, inv, z, g);
    else if constexpr (OUT == LQ_I16) return quant_store<CodeI16>(t, inv, z, g);
    else return quant_store<CodeU8S8>(t, inv, z, g);
}

// One-byte codes take 256 values: their outputs are tabulated once per workgroup in LDS (by
// the same function, so bit-identical) and each element becomes one table read.
template <int IN>
constexpr bool kActLut = IN == LQ_I8 || IN == LQ_U8 || IN == LQ_U8S8;

template <int IN, int OUT>
__global__ __launch_bounds__(kActBlock) void act_kernel(ActArgs a) {
    using TI = typename ElemOf<IN>::type;
    using TO = typename ElemOf<OUT>::type;
    constexpr int WIDE = sizeof(TI) > sizeof(TO) ? sizeof(TI) : sizeof(TO);
    constexpr int E = 16 / WIDE;
    constexpr int U = 8;  // groups in flight per thread
    using VI = typename RawVec<E * sizeof(TI)>::type;
    using VO = typename RawVec<E * sizeof(TO)>::type;
    __shared__ TO lut[kActLut<IN> ? 256 : 1];

    const float sx = a.x_scale ? a.x_scale[0] : 1.0f, zx = a.x_zp ? a.x_zp[0] : 0.0f;
    float inv = 1.0f, z = 0.0f;
    if (OUT != LQ_F32) {
        inv = 1.0f / a.out_scale[0];
        z = a.out_zp ? a.out_zp[0] : 0.0f;
    }
    auto f = [&](TI v) __attribute__((always_inline)) {
        return act_out<OUT>(act_apply(a.op, act_in<IN>(v, sx, zx), a.param), inv, z, a.g);
    };
    if constexpr (kActLut<IN>) {
        static_assert(kActBlock == 256, "one table entry per thread");
        lut[threadIdx.x] = f((TI)(uint8_t)threadIdx.x);
        __syncthreads();
    }
    auto g = [&](TI v) __attribute__((always_inline)) {
        if constexpr (kActLut<IN>) return lut[(uint8_t)v];
        else return f(v);
    };
    const TI* x = static_cast<const TI*>(a.x);
    TO* y = static_cast<TO*>(a.y);
    const int64_t groups = a.vec ? a.n / E : 0;
    // contiguous run of groups per workgroup
    const int64_t per = (groups + gridDim.x - 1) / gridDim.x;
    const int64_t g0 = (int64_t)blockIdx.x * per, g1 = min(groups, g0 + per);
    auto one = [&](int64_t gi, const VI& raw) __attribute__((always_inline)) {
        TI xin[E];
        __builtin_memcpy(xin, &raw, sizeof(raw));
        TO out[E];
#pragma unroll
        for (int e = 0; e < E; ++e) out[e] = g(xin[e]);
        VO ro;
        __builtin_memcpy(&ro, out, sizeof(ro));
        *reinterpret_cast<VO*>(y + gi * E) = ro;
    };
    const VI* xv = reinterpret_cast<const VI*>(x);
    int64_t gi = g0 + threadIdx.x;
    for (; gi + (U - 1) * kActBlock < g1; gi += U * kActBlock) {
        VI raw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) raw[u] = __builtin_nontemporal_load(&xv[gi + u * kActBlock]);
#pragma unroll
        for (int u = 0; u < U; ++u) one(gi + u * kActBlock, raw[u]);
    }
    for (; gi < g1; gi += kActBlock) one(gi, __builtin_nontemporal_load(&xv[gi]));
    // elements past the last full group (all of them when misaligned), one per thread
    const int64_t rest0 = groups * E;
    for (int64_t i = rest0 + (int64_t)blockIdx.x * kActBlock + threadIdx.x; i < a.n; i += (int64_t)gridDim.x * kActBlock)
        y[i] = g(x[i]);
}

static bool act_type_ok(int t) { return t == LQ_F32 || t == LQ_I8 || t == LQ_U8 || t == LQ_I16 || t == LQ_U8S8; }
static int act_bytes(int t) { return t == LQ_F32 ? 4 : t == LQ_I16 ? 2 : 1; }

template <int IN>
static void act_launch_out(int out_type, dim3 grid, hipStream_t st, const ActArgs& a) {
    switch (out_type) {
        case LQ_F32: hipLaunchKernelGGL((act_kernel<IN, LQ_F32>), grid, dim3(kActBlock), 0, st, a); break;
        case LQ_I8: hipLaunchKernelGGL((act_kernel<IN, LQ_I8>), grid, dim3(kActBlock), 0, st, a); break;
        case LQ_U8: hipLaunchKernelGGL((act_kernel<IN, LQ_U8>), grid, dim3(kActBlock), 0, st, a); break;
        case LQ_I16: hipLaunchKernelGGL((act_kernel<IN, LQ_I16>), grid, dim3(kActBlock), 0, st, a); break;
        default: hipLaunchKernelGGL((act_kernel<IN, LQ_U8S8>), grid, dim3(kActBlock), 0, st, a); break;
    }
}

}  // namespace lq

using namespace lq;

extern "C" {

int lq_qact(int op, const void* d_x, int x_type, const float* d_x_scale, const float* d_x_zero_point,
            int64_t n, float param, const float* d_out_scale, const float* d_out_zero_point, int qmin,
            int qmax, int out_type, void* d_y, void* stream) {
    LQ_REQUIRE(op >= LQ_ACT_SIGMOID && op <= LQ_ACT_LEAKY_RELU, "lq_qact: bad op");
    LQ_REQUIRE(n >= 0, "lq_qact: n < 0");
    if (n == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y, "lq_qact: NULL input or output");
    LQ_REQUIRE(act_type_ok(x_type) && act_type_ok(out_type), "lq_qact: unsupported element type");
    LQ_REQUIRE(x_type == LQ_F32 || d_x_scale, "lq_qact: code input needs its scale");
    if (out_type != LQ_F32) {
        LQ_REQUIRE(d_out_scale, "lq_qact: quantized output needs the output scale");
        LQ_REQUIRE(qmax >= qmin, "lq_qact: qmax < qmin");
    }
    const int wide = act_bytes(x_type) > act_bytes(out_type) ? act_bytes(x_type) : act_bytes(out_type);
    const int E = 16 / wide;
    const uintptr_t mx = (uintptr_t)E * act_bytes(x_type) - 1, my = (uintptr_t)E * act_bytes(out_type) - 1;
    const bool vec = ((uintptr_t)d_x & mx) == 0 && ((uintptr_t)d_y & my) == 0;
    ActArgs a{op, d_x, x_type == LQ_F32 ? nullptr : d_x_scale, x_type == LQ_F32 ? nullptr : d_x_zero_point,
              n, param, d_out_scale, d_out_zero_point, make_grid(qmin, qmax), d_y, vec ? 1 : 0};
    // a few groups per thread; up to 32 workgroups per CU to keep enough loads in flight
    const int64_t units = vec ? n / E : n;
    int64_t blocks = (units + 4 * kActBlock - 1) / (4 * kActBlock);
    if (blocks > 8192) blocks = 8192;
    if (blocks < 1) blocks = 1;
    const dim3 grid((unsigned)blocks);
    hipStream_t st = as_stream(stream);
    switch (x_type) {
        case LQ_F32: act_launch_out<LQ_F32>(out_type, grid, st, a); break;
        case LQ_I8: act_launch_out<LQ_I8>(out_type, grid, st, a); break;
        case LQ_U8: act_launch_out<LQ_U8>(out_type, grid, st, a); break;
        case LQ_I16: act_launch_out<LQ_I16>(out_type, grid, st, a); break;
        default: act_launch_out<LQ_U8S8>(out_type, grid, st, a); break;
    }
    return launch_status("lq_qact");
}

}  // extern "C"
