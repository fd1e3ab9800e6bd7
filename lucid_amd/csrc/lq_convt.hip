// lq_convt.hip -- the stride expansion of a transposed convolution.
//
// conv_transpose2d(x, W, stride s, padding p, output_padding q, dilation d) equals a stride-1
// convolution with dilation d of the input expanded by s -- x at every s-th position, the
// zero value in between -- padded by d (k - 1) - p (plus q at the bottom / right), with the
// kernel flipped and its two channel axes swapped (lucid/nn/functional/conv.py
// conv_transpose2d; the direct form is y[n, co, ih s - p + kh d, iw s - p + kw d] +=
// x[n, ci, ih, iw] W[ci, co, kh, kw]).  The quantized layer reuses the int8 implicit-GEMM
// convolution this way; this kernel writes the expanded input, whose gaps hold the
// activation zero point (codes) or 0.0 (floats), so they add exactly nothing.
#include <hip/hip_runtime.h>

#include "lq_internal.h"

namespace lq {

// The gap value: 0.0 for floats; for codes the code of real 0, the zero point read from the
// device (minus 128 for the LQ_U8S8 storage form).
template <typename T>
__global__ __launch_bounds__(256) void stride_expand_kernel(const T* __restrict__ x, int64_t planes, int H, int W,
                                                            int sh, int sw, const float* zp, int zp_shift,
                                                            T* __restrict__ y) {
    const int Hu = (H - 1) * sh + 1, Wu = (W - 1) * sw + 1;
    T fill = T(0);
    if constexpr (sizeof(T) == 1) fill = (T)min(max((zp ? (int)zp[0] : 0) - zp_shift, -128), 127);
    const int64_t total = planes * Hu * Wu;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int w = (int)(i % Wu);
        const int64_t t = i / Wu;
        const int h = (int)(t % Hu);
        const int64_t pl = t / Hu;
        T v = fill;
        if (h % sh == 0 && w % sw == 0) v = x[(pl * H + h / sh) * W + w / sw];
        y[i] = v;
    }
}

}  // namespace lq

using namespace lq;

extern "C" {

int lq_stride_expand(const void* d_x, int elem_type, int64_t planes, int64_t H, int64_t W, int stride_h,
                     int stride_w, const float* d_zero_point, void* d_y, void* stream) {
    LQ_REQUIRE(elem_type == LQ_F32 || elem_type == LQ_I8 || elem_type == LQ_U8S8, "lq_stride_expand: element type must be "
                                                                                   "LQ_F32, LQ_I8 or LQ_U8S8");
    LQ_REQUIRE(planes >= 0 && H >= 1 && W >= 1 && stride_h >= 1 && stride_w >= 1 && H < (1 << 28) && W < (1 << 28),
               "lq_stride_expand: bad shape");
    const int64_t total = planes * ((H - 1) * stride_h + 1) * ((W - 1) * stride_w + 1);
    if (total == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y, "lq_stride_expand: NULL pointer");
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipStream_t st = as_stream(stream);
    if (elem_type == LQ_F32) {
        hipLaunchKernelGGL(stride_expand_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, st,
                           static_cast<const float*>(d_x), planes, (int)H, (int)W, stride_h, stride_w, nullptr, 0,
                           static_cast<float*>(d_y));
    } else {
        hipLaunchKernelGGL(stride_expand_kernel<int8_t>, dim3((unsigned)blocks), dim3(256), 0, st,
                           static_cast<const int8_t*>(d_x), planes, (int)H, (int)W, stride_h, stride_w,
                           d_zero_point, elem_type == LQ_U8S8 ? 128 : 0, static_cast<int8_t*>(d_y));
    }
    return launch_status("lq_stride_expand");
}

}  // extern "C"
