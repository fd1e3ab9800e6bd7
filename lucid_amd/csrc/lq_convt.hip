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

// ------------------------------------------------------------------ 3-D convolutions
//
// A 3-D convolution is a 2-D one over depth-stacked channels: output depth od of batch n
// reads, for each kernel depth kd, the input slice at depth e = od s - p + kd d, so the
// gathered input [N OD, groups, KD, C/groups, H, W] (slice kd of group g at channel
// (g KD + kd) C/groups + c) convolved in 2-D with the kernel rearranged to
// [Cout, KD C/groups, KH, KW] sums exactly the products of the 3-D convolution; for codes the
// int32 sums are the same integers, so the requantized outputs are the same codes.  A
// transposed 3-D convolution expands the depth axis by its stride: e indexes the expanded
// axis, whose positions e % expand != 0 hold the zero value.  Depth padding: the zero value,
// or the reflect / replicate / circular source (expand == 1).
__device__ __forceinline__ int64_t depth_source(int64_t e, int64_t D, int64_t expand, int mode) {
    if (expand > 1) {
        if (e < 0 || e % expand) return -1;
        e /= expand;
        return e < D ? e : -1;
    }
    if (e >= 0 && e < D) return e;
    if (mode == 0) return -1;
    if (mode == 1) {  // reflect (edge not repeated)
        if (D == 1) return 0;
        const int64_t period = 2 * (D - 1);
        int64_t r = e % period;
        if (r < 0) r += period;
        return r < D ? r : period - r;
    }
    if (mode == 2) return e < 0 ? 0 : D - 1;  // replicate
    int64_t r = e % D;                         // circular
    return r < 0 ? r + D : r;
}

template <typename T>
__global__ __launch_bounds__(256) void depth_gather_kernel(const T* __restrict__ x, int64_t N, int64_t C, int64_t D,
                                                           int64_t HW, int64_t groups, int64_t KD, int64_t OD,
                                                           int64_t stride, int64_t pad, int64_t dil, int64_t expand,
                                                           int mode, const float* zp, int zp_shift, T* __restrict__ y) {
    T fill = T(0);
    if constexpr (sizeof(T) == 1) fill = (T)min(max((zp ? (int)zp[0] : 0) - zp_shift, -128), 127);
    const int64_t Cg = C / groups;
    const int64_t total = N * OD * groups * KD * Cg * HW;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t hw = i % HW;
        int64_t t = i / HW;
        const int64_t c = t % Cg;
        t /= Cg;
        const int64_t kd = t % KD;
        t /= KD;
        const int64_t g = t % groups;
        t /= groups;
        const int64_t od = t % OD;
        const int64_t n = t / OD;
        const int64_t id = depth_source(od * stride - pad + kd * dil, D, expand, mode);
        y[i] = id < 0 ? fill : x[((n * C + g * Cg + c) * D + id) * HW + hw];
    }
}

// y[a][c][b][p] = x[a][b][c][p]: swaps the two middle axes of a 4-D view (a 2-D convolution's
// [N, OD, Cout, OH OW] output into NCDHW, or a kernel's [Cout, C, KD, KH KW] into the gathered
// [Cout, KD, C, KH KW] order), in units of U bytes.
template <typename U>
__global__ __launch_bounds__(256) void permute_0213_kernel(const U* __restrict__ x, int64_t A, int64_t B, int64_t C,
                                                           int64_t P, U* __restrict__ y) {
    const int64_t total = A * B * C * P;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t p = i % P;
        int64_t t = i / P;
        const int64_t b = t % B;  // output index order a, c, b, p
        t /= B;
        const int64_t c = t % C;
        const int64_t a = t / C;
        y[i] = x[((a * B + b) * C + c) * P + p];
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

int lq_depth_gather(const void* d_x, int elem_type, int64_t N, int64_t C, int64_t D, int64_t HW, int64_t groups,
                    int64_t KD, int64_t OD, int64_t stride, int64_t pad, int64_t dilation, int64_t expand,
                    int pad_mode, const float* d_zero_point, void* d_y, void* stream) {
    LQ_REQUIRE(elem_type == LQ_F32 || elem_type == LQ_I8 || elem_type == LQ_U8S8, "lq_depth_gather: element type must "
                                                                                   "be LQ_F32, LQ_I8 or LQ_U8S8");
    LQ_REQUIRE(N >= 0 && C >= 1 && D >= 1 && HW >= 1 && groups >= 1 && C % groups == 0 && KD >= 1 && OD >= 0 &&
                   stride >= 1 && dilation >= 1 && expand >= 1 && pad_mode >= 0 && pad_mode <= 3,
               "lq_depth_gather: bad shape");
    LQ_REQUIRE(expand == 1 || pad_mode == 0, "lq_depth_gather: an expanded depth axis pads with zeros only");
    LQ_REQUIRE(pad_mode == 0 || pad < D, "lq_depth_gather: reflect / circular depth padding must be below D");
    const int64_t total = N * OD * KD * C * HW;
    if (total == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y, "lq_depth_gather: NULL pointer");
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipStream_t st = as_stream(stream);
    if (elem_type == LQ_F32)
        hipLaunchKernelGGL(depth_gather_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, st,
                           static_cast<const float*>(d_x), N, C, D, HW, groups, KD, OD, stride, pad, dilation, expand,
                           pad_mode, nullptr, 0, static_cast<float*>(d_y));
    else
        hipLaunchKernelGGL(depth_gather_kernel<int8_t>, dim3((unsigned)blocks), dim3(256), 0, st,
                           static_cast<const int8_t*>(d_x), N, C, D, HW, groups, KD, OD, stride, pad, dilation, expand,
                           pad_mode, d_zero_point, elem_type == LQ_U8S8 ? 128 : 0, static_cast<int8_t*>(d_y));
    return launch_status("lq_depth_gather");
}

int lq_permute_0213(const void* d_x, int elem_bytes, int64_t A, int64_t B, int64_t C, int64_t P, void* d_y,
                    void* stream) {
    LQ_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4, "lq_permute_0213: element size 1, 2 or 4");
    LQ_REQUIRE(A >= 0 && B >= 0 && C >= 0 && P >= 0, "lq_permute_0213: bad shape");
    const int64_t total = A * B * C * P;
    if (total == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y && d_x != d_y, "lq_permute_0213: NULL or aliased pointer");
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipStream_t st = as_stream(stream);
    if (elem_bytes == 1)
        hipLaunchKernelGGL(permute_0213_kernel<uint8_t>, dim3((unsigned)blocks), dim3(256), 0, st,
                           static_cast<const uint8_t*>(d_x), A, B, C, P, static_cast<uint8_t*>(d_y));
    else if (elem_bytes == 2)
        hipLaunchKernelGGL(permute_0213_kernel<uint16_t>, dim3((unsigned)blocks), dim3(256), 0, st,
                           static_cast<const uint16_t*>(d_x), A, B, C, P, static_cast<uint16_t*>(d_y));
    else
        hipLaunchKernelGGL(permute_0213_kernel<uint32_t>, dim3((unsigned)blocks), dim3(256), 0, st,
                           static_cast<const uint32_t*>(d_x), A, B, C, P, static_cast<uint32_t*>(d_y));
    return launch_status("lq_permute_0213");
}

}  // extern "C"
