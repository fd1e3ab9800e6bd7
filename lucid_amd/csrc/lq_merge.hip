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
