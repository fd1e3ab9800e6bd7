// lq_hist.hip -- the histogram half of Lucid's HistogramObserver on the GPU.
//
// HistogramObserver.forward (lucid/quantization/observer.py:850-870) keeps a `bins`-bucket
// float32 histogram over its running [min, max].  Each batch is counted with Lucid's
// histc (lucid/_ops/_adapters.py:1256-1279 -> lucid/_C/ops/composite/Stats.cpp:48-96 ->
// lucid/_C/backend/cpu/methods/Reduction.cpp:839-884): in double precision,
// step = (hi - lo) / bins, an element v lands in bin trunc((v - lo) / step), the top edge
// in the last bin; elements outside [lo, hi] and NaN (the adapter maps NaN below the range)
// are skipped.  The double counts become float32 and are added to the running histogram
// in float32.  When the running range widens, the stored histogram is first moved onto the
// new bins (observer.py:826-848): float32 bin centers, a float32 index, truncation, and a
// scatter_add in source order.
//
// lq_histc_f32: per-block LDS counts (uint32, exact), one atomic flush per non-empty bin,
// then a finalize pass that converts and adds in float32.  lq_hist_rebin_f32: one
// workgroup; source bin i maps to a target index that never decreases with i, so each
// target bin receives one contiguous run of sources, summed in source order -- the same
// float32 additions as the sequential scatter_add.
#include <hip/hip_runtime.h>

#include "lq_internal.h"

namespace lq {

constexpr int kHistBlock = 256;
constexpr int64_t kHistLdsBins = 8192;   // 32 KB of LDS counts per block
constexpr int64_t kRebinMaxBins = 16384; // target indices of one rebin held in LDS

__global__ __launch_bounds__(kHistBlock) void hist_clear_kernel(uint32_t* cnt, int64_t bins) {
    for (int64_t b = (int64_t)blockIdx.x * kHistBlock + threadIdx.x; b < bins; b += (int64_t)gridDim.x * kHistBlock)
        cnt[b] = 0u;
}

__device__ __forceinline__ int64_t hist_bin(float v, double lo, double hi, double step, int64_t bins) {
    const double d = (double)v;
    if (d != d || d < lo || d > hi) return -1;
    int64_t b = (int64_t)((d - lo) / step);
    return b >= bins ? bins - 1 : b;
}

// Counts of x[n] into cnt[bins] (uint32).  Each block walks one contiguous run of x.
template <bool LDS>
__global__ __launch_bounds__(kHistBlock) void hist_count_kernel(const float* __restrict__ x, int64_t n, double lo,
                                                                double hi, double step, int64_t bins,
                                                                uint32_t* __restrict__ cnt) {
    extern __shared__ uint32_t sh[];
    if (LDS) {
        for (int64_t b = threadIdx.x; b < bins; b += kHistBlock) sh[b] = 0u;
        __syncthreads();
    }
    const int64_t chunk = ((n + gridDim.x - 1) / gridDim.x + kHistBlock - 1) / kHistBlock * kHistBlock;
    const int64_t b0 = min(n, (int64_t)blockIdx.x * chunk), b1 = min(n, b0 + chunk);
    for (int64_t i = b0 + threadIdx.x; i < b1; i += kHistBlock) {
        const int64_t b = hist_bin(x[i], lo, hi, step, bins);
        if (b >= 0) {
            if (LDS) atomicAdd(&sh[b], 1u);
            else atomicAdd(&cnt[b], 1u);
        }
    }
    if (LDS) {
        __syncthreads();
        for (int64_t b = threadIdx.x; b < bins; b += kHistBlock)
            if (sh[b]) atomicAdd(&cnt[b], sh[b]);
    }
}

// hist[b] = fl32(float(cnt[b]) + hist[b]) (accumulate) or float(cnt[b]).
__global__ __launch_bounds__(kHistBlock) void hist_finalize_kernel(const uint32_t* __restrict__ cnt, int64_t bins,
                                                                   int accumulate, float* __restrict__ hist) {
    for (int64_t b = (int64_t)blockIdx.x * kHistBlock + threadIdx.x; b < bins; b += (int64_t)gridDim.x * kHistBlock) {
        const float c = (float)cnt[b];
        hist[b] = accumulate ? c + hist[b] : c;
    }
}

// out[j] = sum, in source order, of hist[i] over the sources with target j, where
// target(i) = trunc(clip(fl32(fl32(old_min + fl32((i + 0.5) * old_w)) - new_min) / new_w,
//                        0, bins - 1)), every operation in float32.
__global__ __launch_bounds__(1024) void hist_rebin_kernel(const float* __restrict__ hist, int64_t bins, float old_min,
                                                          float old_w, float new_min, float new_w,
                                                          float* __restrict__ out) {
    extern __shared__ int32_t dst[];
    const float top = (float)(bins - 1);
    for (int64_t i = threadIdx.x; i < bins; i += blockDim.x) {
        const float t = (float)i + 0.5f;
        const float c = old_min + t * old_w;
        float r = (c - new_min) / new_w;
        r = r < 0.0f ? 0.0f : (r > top ? top : r);
        if (r != r) r = 0.0f;  // a zero-width target range (never passed by the observer)
        dst[i] = (int32_t)r;
    }
    __syncthreads();
    for (int64_t j = threadIdx.x; j < bins; j += blockDim.x) {
        // first source with target >= j, then the run with target == j
        int64_t a = 0, e = bins;
        while (a < e) {
            const int64_t m = (a + e) >> 1;
            if (dst[m] < j) a = m + 1;
            else e = m;
        }
        float s = 0.0f;
        for (int64_t i = a; i < bins && dst[i] == j; ++i) s = s + hist[i];
        out[j] = s;
    }
}

}  // namespace lq

using namespace lq;

extern "C" {

size_t lq_histc_workspace_size(int64_t bins) { return bins > 0 ? (size_t)bins * sizeof(uint32_t) : 0; }

int lq_histc_f32(const float* d_x, int64_t n, int64_t bins, double lo, double hi, int accumulate, float* d_hist,
                 void* d_workspace, size_t workspace_bytes, void* stream) {
    LQ_REQUIRE(n >= 0 && bins > 0, "lq_histc_f32: need n >= 0 and bins > 0");
    LQ_REQUIRE(n == 0 || d_x, "lq_histc_f32: NULL input");
    LQ_REQUIRE(d_hist, "lq_histc_f32: NULL histogram");
    LQ_REQUIRE(hi > lo, "lq_histc_f32: need hi > lo");
    LQ_REQUIRE(d_workspace && workspace_bytes >= lq_histc_workspace_size(bins), "lq_histc_f32: workspace too small");
    hipStream_t st = as_stream(stream);
    uint32_t* cnt = static_cast<uint32_t*>(d_workspace);
    const unsigned gb = (unsigned)std::min<int64_t>((bins + kHistBlock - 1) / kHistBlock, 1024);
    hipLaunchKernelGGL(hist_clear_kernel, dim3(gb), dim3(kHistBlock), 0, st, cnt, bins);
    if (n > 0) {
        const double step = (hi - lo) / (double)bins;
        int64_t blocks = (n + 4 * kHistBlock - 1) / (4 * kHistBlock);
        if (blocks > 2048) blocks = 2048;
        if (bins <= kHistLdsBins)
            hipLaunchKernelGGL(hist_count_kernel<true>, dim3((unsigned)blocks), dim3(kHistBlock),
                               (size_t)bins * sizeof(uint32_t), st, d_x, n, lo, hi, step, bins, cnt);
        else
            hipLaunchKernelGGL(hist_count_kernel<false>, dim3((unsigned)blocks), dim3(kHistBlock), 0, st, d_x, n, lo,
                               hi, step, bins, cnt);
    }
    hipLaunchKernelGGL(hist_finalize_kernel, dim3(gb), dim3(kHistBlock), 0, st, cnt, bins, accumulate, d_hist);
    return launch_status("lq_histc_f32");
}

int lq_hist_rebin_f32(const float* d_hist, int64_t bins, float old_min, float old_width, float new_min,
                      float new_width, float* d_out, void* stream) {
    LQ_REQUIRE(bins > 0 && bins <= kRebinMaxBins, "lq_hist_rebin_f32: bins must be in [1, 16384]");
    LQ_REQUIRE(d_hist && d_out && d_hist != d_out, "lq_hist_rebin_f32: need distinct input and output");
    hipLaunchKernelGGL(hist_rebin_kernel, dim3(1), dim3(1024), (size_t)bins * sizeof(int32_t), as_stream(stream),
                       d_hist, bins, old_min, old_width, new_min, new_width, d_out);
    return launch_status("lq_hist_rebin_f32");
}

}  // extern "C"
