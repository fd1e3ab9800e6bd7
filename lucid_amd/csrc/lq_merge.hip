// lq_merge.hip -- the element-wise merges of FloatFunctional / QFunctional.
//
// A residual network quantizes end to end only if its skip-adds (and concatenations) are
// requantized onto one calibrated grid: Lucid's FloatFunctional observes the float merge
// during calibration and QFunctional fake-quantizes it afterwards
// (lucid/nn/quantized/functional_module.py:95-235).  Here one kernel does the whole merge:
// it reads each operand either as float32 or as integer codes with their own per-tensor
// grid (dequantized as fl32(fl32(float(c) - z) * s), lucid/quantization/_functional.py:293),
// applies the float32 op (x + y, x * y, x + scalar, x * scalar, or a copy for cat), an
// optional ReLU (y <= 0 -> +0, NaN passes), and writes either the float result or its codes
// on the output grid (clip(rne(t * fl32(1 / S)) + Z), stored in the integer domain).  A
// code-backed activation therefore never materializes its floats: an int8 skip-add moves
// 3 bytes per element.
#include <hip/hip_runtime.h>

#include "lq_internal.h"

namespace lq {

constexpr int kMergeBlock = 256;

__device__ __forceinline__ float merge_load(const void* p, int type, int64_t i, float s, float z) {
    float c;
    switch (type) {
        case LQ_F32:
            return static_cast<const float*>(p)[i];
        case LQ_I8:
            c = (float)static_cast<const int8_t*>(p)[i];
            break;
        case LQ_U8:
            c = (float)static_cast<const uint8_t*>(p)[i];
            break;
        case LQ_I16:
            c = (float)static_cast<const int16_t*>(p)[i];
            break;
        default:  // LQ_U8S8: the unsigned code c stored as c - 128
            c = (float)((int)static_cast<const int8_t*>(p)[i] + 128);
            break;
    }
    const float d = c - z;
    return d * s;
}

struct MergeArgs {
    int op;
    const void* a;
    int a_type;
    const float* a_scale;
    const float* a_zp;
    const void* b;
    int b_type;
    const float* b_scale;
    const float* b_zp;
    float scalar;
    int64_t rows, cols, ld_out;
    const float* out_scale;
    const float* out_zp;
    Grid g;
    int relu;
    void* out;
};

// One element per thread per step; blockIdx.y walks rows, blockIdx.x a contiguous run of
// columns.  OUT is LQ_F32 (the float merge) or a code type (the requantized merge).
template <int OUT>
__global__ __launch_bounds__(kMergeBlock) void merge_kernel(MergeArgs m) {
    const float sa = m.a_scale ? m.a_scale[0] : 1.0f, za = m.a_zp ? m.a_zp[0] : 0.0f;
    const float sb = m.b_scale ? m.b_scale[0] : 1.0f, zb = m.b_zp ? m.b_zp[0] : 0.0f;
    float s = 1.0f, inv = 1.0f, z = 0.0f;
    if (OUT != LQ_F32) {
        s = m.out_scale[0];
        inv = 1.0f / s;
        z = m.out_zp ? m.out_zp[0] : 0.0f;
    }
    const int64_t chunk = ((m.cols + gridDim.x - 1) / gridDim.x + kMergeBlock - 1) / kMergeBlock * kMergeBlock;
    const int64_t c0 = min(m.cols, (int64_t)blockIdx.x * chunk), c1 = min(m.cols, c0 + chunk);
    for (int64_t r = blockIdx.y; r < m.rows; r += gridDim.y) {
        for (int64_t c = c0 + threadIdx.x; c < c1; c += kMergeBlock) {
            const int64_t i = r * m.cols + c;
            const float a = merge_load(m.a, m.a_type, i, sa, za);
            float t;
            switch (m.op) {
                case LQ_MERGE_ADD:
                    t = a + merge_load(m.b, m.b_type, i, sb, zb);
                    break;
                case LQ_MERGE_MUL:
                    t = a * merge_load(m.b, m.b_type, i, sb, zb);
                    break;
                case LQ_MERGE_ADD_SCALAR:
                    t = a + m.scalar;
                    break;
                case LQ_MERGE_MUL_SCALAR:
                    t = a * m.scalar;
                    break;
                default:  // LQ_MERGE_COPY
                    t = a;
                    break;
            }
            if (m.relu) t = (t <= 0.0f) ? 0.0f : t;
            const int64_t o = r * m.ld_out + c;
            if (OUT == LQ_F32) static_cast<float*>(m.out)[o] = t;
            else if (OUT == LQ_I8) static_cast<int8_t*>(m.out)[o] = quant_store<CodeI8>(t, inv, z, m.g);
            else if (OUT == LQ_U8) static_cast<uint8_t*>(m.out)[o] = quant_store<CodeU8>(t, inv, z, m.g);
            else if (OUT == LQ_I16) static_cast<int16_t*>(m.out)[o] = quant_store<CodeI16>(t, inv, z, m.g);
            else static_cast<int8_t*>(m.out)[o] = quant_store<CodeU8S8>(t, inv, z, m.g);
        }
    }
}

// Byte codes, contiguous operands and output, 16 elements (one 16-byte load of each operand,
// one 16-byte store) per thread per step: the residual adds of a quantized network.  Each
// element goes through the same operations as merge_kernel (merge_load, the op, ReLU,
// quant_store), so the two paths agree bit for bit.
template <int T>
__device__ __forceinline__ float byte_code(uint32_t b) {  // b: the stored byte in bits 0-7
    if constexpr (T == LQ_I8) return (float)(int)(int8_t)(uint8_t)b;
    else if constexpr (T == LQ_U8) return (float)(int)(uint8_t)b;
    else return (float)((int)(int8_t)(uint8_t)b + 128);  // LQ_U8S8
}

template <int OUT>
__device__ __forceinline__ uint32_t byte_store(float t, float inv, float z, const Grid& g) {
    if constexpr (OUT == LQ_I8) return (uint8_t)quant_store<CodeI8>(t, inv, z, g);
    else if constexpr (OUT == LQ_U8) return (uint8_t)quant_store<CodeU8>(t, inv, z, g);
    else return (uint8_t)quant_store<CodeU8S8>(t, inv, z, g);
}

template <int AT, int BT, int OUT, bool MUL>
__global__ __launch_bounds__(kMergeBlock) void merge_bytes16_kernel(MergeArgs m, int64_t n16) {
    const float sa = m.a_scale[0], za = m.a_zp ? m.a_zp[0] : 0.0f;
    const float sb = m.b_scale[0], zb = m.b_zp ? m.b_zp[0] : 0.0f;
    const float s = m.out_scale[0], inv = 1.0f / s, z = m.out_zp ? m.out_zp[0] : 0.0f;
    const vu4* A = static_cast<const vu4*>(m.a);
    const vu4* B = static_cast<const vu4*>(m.b);
    vu4* Y = static_cast<vu4*>(m.out);
    for (int64_t v = (int64_t)blockIdx.x * kMergeBlock + threadIdx.x; v < n16; v += (int64_t)gridDim.x * kMergeBlock) {
        const vu4 xa = A[v], xb = B[v];
        vu4 y;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t o = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float a = (byte_code<AT>(xa[w] >> (8 * e)) - za) * sa;
                const float b = (byte_code<BT>(xb[w] >> (8 * e)) - zb) * sb;
                float t = MUL ? a * b : a + b;
                if (m.relu) t = (t <= 0.0f) ? 0.0f : t;
                o |= byte_store<OUT>(t, inv, z, m.g) << (8 * e);
            }
            y[w] = o;
        }
        Y[v] = y;
    }
}

static bool byte_code_type(int t) { return t == LQ_I8 || t == LQ_U8 || t == LQ_U8S8; }

static bool merge_type_ok(int t) { return t == LQ_F32 || t == LQ_I8 || t == LQ_U8 || t == LQ_I16 || t == LQ_U8S8; }

}  // namespace lq

using namespace lq;

extern "C" {

int lq_qmerge(int op, const void* d_a, int a_type, const float* d_a_scale, const float* d_a_zero_point,
              const void* d_b, int b_type, const float* d_b_scale, const float* d_b_zero_point, float scalar,
              int64_t rows, int64_t cols, int64_t ld_out, const float* d_out_scale,
              const float* d_out_zero_point, int qmin, int qmax, int flags, int out_type, void* d_out,
              void* stream) {
    LQ_REQUIRE(op >= LQ_MERGE_ADD && op <= LQ_MERGE_COPY, "lq_qmerge: bad op");
    LQ_REQUIRE(rows >= 0 && cols >= 0 && ld_out >= cols, "lq_qmerge: need rows, cols >= 0 and ld_out >= cols");
    if (rows == 0 || cols == 0) return LQ_OK;
    LQ_REQUIRE(d_a && d_out, "lq_qmerge: NULL operand or output");
    LQ_REQUIRE(merge_type_ok(a_type) && merge_type_ok(out_type), "lq_qmerge: unsupported element type");
    LQ_REQUIRE(a_type == LQ_F32 || d_a_scale, "lq_qmerge: code operand a needs its scale");
    const bool binary = op == LQ_MERGE_ADD || op == LQ_MERGE_MUL;
    if (binary) {
        LQ_REQUIRE(d_b && merge_type_ok(b_type), "lq_qmerge: bad operand b");
        LQ_REQUIRE(b_type == LQ_F32 || d_b_scale, "lq_qmerge: code operand b needs its scale");
    }
    if (out_type != LQ_F32) {
        LQ_REQUIRE(d_out_scale, "lq_qmerge: requantized output needs the output scale");
        LQ_REQUIRE(qmax >= qmin, "lq_qmerge: qmax < qmin");
    }
    LQ_REQUIRE((flags & ~LQ_EPI_RELU) == 0, "lq_qmerge: unknown flag");
    MergeArgs m{op, d_a, a_type, a_type == LQ_F32 ? nullptr : d_a_scale, d_a_zero_point,
                binary ? d_b : nullptr, b_type, binary && b_type != LQ_F32 ? d_b_scale : nullptr, d_b_zero_point,
                scalar, rows, cols, ld_out, d_out_scale, d_out_zero_point, make_grid(qmin, qmax),
                (flags & LQ_EPI_RELU) != 0, d_out};
    hipStream_t st0 = as_stream(stream);
    const int64_t n = rows * cols;
    if (binary && (ld_out == cols || rows == 1) && byte_code_type(a_type) && a_type == b_type &&
        byte_code_type(out_type) && n % 16 == 0 &&
        ((reinterpret_cast<uintptr_t>(d_a) | reinterpret_cast<uintptr_t>(d_b) | reinterpret_cast<uintptr_t>(d_out)) &
         15) == 0) {
        const int64_t n16 = n / 16;
        int64_t blocks = (n16 + kMergeBlock - 1) / kMergeBlock;
        if (blocks > 8192) blocks = 8192;
        const dim3 g16((unsigned)blocks);
#define LQ_MERGE16(AT, OT)                                                                                 \
    do {                                                                                                   \
        if (op == LQ_MERGE_ADD) hipLaunchKernelGGL((merge_bytes16_kernel<AT, AT, OT, false>), g16, dim3(kMergeBlock), 0, st0, m, n16); \
        else hipLaunchKernelGGL((merge_bytes16_kernel<AT, AT, OT, true>), g16, dim3(kMergeBlock), 0, st0, m, n16);  \
    } while (0)
#define LQ_MERGE16_OUT(AT)                                   \
    do {                                                     \
        if (out_type == LQ_I8) LQ_MERGE16(AT, LQ_I8);        \
        else if (out_type == LQ_U8) LQ_MERGE16(AT, LQ_U8);   \
        else LQ_MERGE16(AT, LQ_U8S8);                        \
    } while (0)
        if (a_type == LQ_I8) LQ_MERGE16_OUT(LQ_I8);
        else if (a_type == LQ_U8) LQ_MERGE16_OUT(LQ_U8);
        else LQ_MERGE16_OUT(LQ_U8S8);
#undef LQ_MERGE16_OUT
#undef LQ_MERGE16
        return launch_status("lq_qmerge");
    }
    int64_t bx = (cols + 4 * kMergeBlock - 1) / (4 * kMergeBlock);
    if (bx > 4096) bx = 4096;
    const int64_t by = rows < 65535 ? rows : 65535;
    const dim3 grid((unsigned)bx, (unsigned)by);
    hipStream_t st = as_stream(stream);
    switch (out_type) {
        case LQ_F32: hipLaunchKernelGGL(merge_kernel<LQ_F32>, grid, dim3(kMergeBlock), 0, st, m); break;
        case LQ_I8: hipLaunchKernelGGL(merge_kernel<LQ_I8>, grid, dim3(kMergeBlock), 0, st, m); break;
        case LQ_U8: hipLaunchKernelGGL(merge_kernel<LQ_U8>, grid, dim3(kMergeBlock), 0, st, m); break;
        case LQ_I16: hipLaunchKernelGGL(merge_kernel<LQ_I16>, grid, dim3(kMergeBlock), 0, st, m); break;
        default: hipLaunchKernelGGL(merge_kernel<LQ_U8S8>, grid, dim3(kMergeBlock), 0, st, m); break;
    }
    return launch_status("lq_qmerge");
}

}  // extern "C"
