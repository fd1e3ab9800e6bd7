// lq_float.hip -- float helper kernels around the quantized path: ReLU, the float Linear
// used to calibrate (run) the float model before convert(), and conversions between float32,
// half and bfloat16 (Lucid's astype between float dtypes).
//
// ReLU follows Lucid's CPU rule `x <= 0 ? 0 : x` (lucid/_C/backend/cpu/Vdsp.cpp vrelu_f32:
// NaN passes, -0 becomes +0).  The float Linear is y = x W^T + b
// (lucid/_C/backend/cpu/methods/Matmul.cpp:80-122); its summation order, like Accelerate's
// sgemm order, is an implementation detail, so only tolerance parity applies to it.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "lq_internal.h"

namespace lq {

__global__ void relu_f32_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        float v = x[i];
        y[i] = (v <= 0.0f) ? 0.0f : v;
    }
}

// One element per thread-iteration; every conversion is exact when widening and rounds to
// nearest even when narrowing (half through v_cvt_f16_f32, bfloat16 on the upper 16 bits).
template <int XT, int YT>
__global__ void cast_kernel(const void* __restrict__ xv, void* __restrict__ yv, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        float v;
        if constexpr (XT == LQ_F32) v = static_cast<const float*>(xv)[i];
        else if constexpr (XT == LQ_F16) v = __half2float(static_cast<const __half*>(xv)[i]);
        else v = bf16_bits_to_f32(static_cast<const uint16_t*>(xv)[i]);
        if constexpr (YT == LQ_F32) static_cast<float*>(yv)[i] = v;
        else if constexpr (YT == LQ_F16) static_cast<__half*>(yv)[i] = f32_to_f16_rn(v);
        else static_cast<uint16_t*>(yv)[i] = f32_to_bf16_bits(v);
    }
}

// 64x64 output tile per 256-thread block, 4x4 outputs per thread, K-steps of 16 via LDS.
constexpr int LT = 64, LK = 16;

__global__ __launch_bounds__(256) void linear_f32_kernel(const float* __restrict__ x, int64_t ldx,
                                                         const float* __restrict__ w, int64_t ldw,
                                                         const float* __restrict__ bias,
                                                         float* __restrict__ y, int64_t ldy,
                                                         int64_t M, int64_t N, int64_t K) {
    __shared__ float xs[LK][LT + 1];
    __shared__ float ws[LK][LT + 1];
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const int64_t m0 = (int64_t)blockIdx.y * LT, n0 = (int64_t)blockIdx.x * LT;
    float acc[4][4] = {};
    for (int64_t k0 = 0; k0 < K; k0 += LK) {
        for (int e = threadIdx.x; e < LT * LK; e += 256) {
            int r = e / LK, kk = e % LK;
            int64_t gm = m0 + r, gn = n0 + r, gk = k0 + kk;
            xs[kk][r] = (gm < M && gk < K) ? x[gm * ldx + gk] : 0.0f;
            ws[kk][r] = (gn < N && gk < K) ? w[gn * ldw + gk] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < LK; ++kk) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a[i] = xs[kk][ty * 4 + i];
                b[i] = ws[kk][tx * 4 + i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int64_t gm = m0 + ty * 4 + i;
        if (gm >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int64_t gn = n0 + tx * 4 + j;
            if (gn >= N) continue;
            float v = acc[i][j];
            if (bias) v = v + bias[gn];
            y[gm * ldy + gn] = v;
        }
    }
}

}  // namespace lq

using namespace lq;

extern "C" {

int lq_cast(const void* d_x, int x_dtype, void* d_y, int y_dtype, int64_t n, void* stream) {
    auto is_float = [](int t) { return t == LQ_F32 || t == LQ_F16 || t == LQ_BF16; };
    LQ_REQUIRE(is_float(x_dtype) && is_float(y_dtype), "lq_cast: types must be LQ_F32, LQ_F16 or LQ_BF16");
    LQ_REQUIRE(n >= 0, "lq_cast: negative count");
    if (n == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y, "lq_cast: NULL pointer");
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
    hipStream_t st = as_stream(stream);
    const dim3 g((unsigned)blocks), b(256);
#define LQ_CAST(X, Y) \
    if (x_dtype == X && y_dtype == Y) hipLaunchKernelGGL((cast_kernel<X, Y>), g, b, 0, st, d_x, d_y, n)
    LQ_CAST(LQ_F32, LQ_F32); LQ_CAST(LQ_F32, LQ_F16); LQ_CAST(LQ_F32, LQ_BF16);
    LQ_CAST(LQ_F16, LQ_F32); LQ_CAST(LQ_F16, LQ_F16); LQ_CAST(LQ_F16, LQ_BF16);
    LQ_CAST(LQ_BF16, LQ_F32); LQ_CAST(LQ_BF16, LQ_F16); LQ_CAST(LQ_BF16, LQ_BF16);
#undef LQ_CAST
    return launch_status("lq_cast");
}

int lq_relu_f32(const float* d_x, float* d_y, int64_t n, void* stream) {
    LQ_REQUIRE(n >= 0, "lq_relu_f32: n < 0");
    if (n == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y, "lq_relu_f32: NULL pointer");
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(relu_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                       d_x, d_y, n);
    return launch_status("lq_relu_f32");
}

int lq_linear_f32(const float* d_x, int64_t ldx, const float* d_w, int64_t ldw,
                  const float* d_bias, float* d_y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                  void* stream) {
    LQ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "lq_linear_f32: negative size");
    if (M == 0 || N == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_w && d_y, "lq_linear_f32: NULL pointer");
    LQ_REQUIRE(ldx >= K && ldw >= K && ldy >= N, "lq_linear_f32: leading dimension too small");
    int64_t gx = (N + LT - 1) / LT, gy = (M + LT - 1) / LT;
    LQ_REQUIRE(gx <= 0x7fffffff && gy <= 65535, "lq_linear_f32: problem too large");
    hipLaunchKernelGGL(linear_f32_kernel, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0,
                       as_stream(stream), d_x, ldx, d_w, ldw, d_bias, d_y, ldy, M, N, K);
    return launch_status("lq_linear_f32");
}

}  // extern "C"
