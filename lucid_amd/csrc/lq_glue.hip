// lq_glue.hip -- the float kernels a dynamically quantized transformer runs between its int8
// Linears (token + position embedding, layer norm, causal
// attention over an fp16 KV cache, GELU, residual adds, greedy argmax).  They follow Lucid's
// float modules (lucid/nn/modules/normalization.py LayerNorm, nn/functional/attention.py
// scaled_dot_product_attention with is_causal, nn/functional/activation.py gelu tanh form);
// their results are compared with float64 restatements within tolerance (their summation
// order is not knowable from the reference either).
//
// Attention.  One workgroup (256 threads) per (batch, head, block of QPB queries): the
// block's queries go to LDS; every thread scores its keys against all QPB queries (fp16
// K rows, fp32 dot products) into an LDS score table; each wave turns two rows into
// softmax weights (max, exp, sum by wave reduction); then each thread accumulates output
// dims from fp16 V rows read coalesced across the 64 lanes.  Query i (absolute position
// pos0 + i) sees keys 0 .. pos0 + i.  KV cache layout [B][H][T_max][hd] fp16.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "lq_internal.h"

namespace lq {
namespace {

constexpr int ATT_THREADS = 256;
constexpr int ATT_MAX_T = 2048;  // keys per query at most (LDS score table)
constexpr int ATT_HD = 64;       // head dim of the kernels below

// The position of the first token: pos0, or *d_pos0 when given (graph replay across decode
// steps), clamped to [0, hi] so every access stays in range.
__device__ __forceinline__ int64_t position(int64_t pos0, const int32_t* d_pos0, int64_t hi) {
    int64_t p = d_pos0 ? (int64_t)d_pos0[0] : pos0;
    return p < 0 ? 0 : (p > hi ? hi : p);
}

__global__ __launch_bounds__(256) void embedding_sum_kernel(const float* __restrict__ tok, const float* __restrict__ pos,
                                                            int64_t npos, int64_t D, const int32_t* __restrict__ tokens,
                                                            int64_t rows, int64_t n, int64_t pos0,
                                                            const int32_t* __restrict__ d_pos0, int64_t vocab,
                                                            float* __restrict__ out) {
    const int64_t r = blockIdx.x;  // token row (b * n + i)
    if (r >= rows) return;
    const int64_t i = r % n;
    pos0 = position(pos0, d_pos0, npos - n);
    int64_t t = tokens[r];
    t = t < 0 ? 0 : (t >= vocab ? vocab - 1 : t);  // ids were validated on the host; clamp keeps reads in range
    const float* a = tok + t * D;
    const float* p = pos + (pos0 + i) * D;
    for (int64_t d = threadIdx.x; d < D; d += blockDim.x) out[r * D + d] = a[d] + p[d];
}

// y = (x - mean) / sqrt(var + eps) [* gamma + beta]: mean and biased variance in float32
// over the row (wave-level tree sums), one workgroup per row.
// RES: the row is first replaced by x + res (the residual add, one rounding per element, each
// element written and read back by the same thread), and the norm runs on the sums: the same
// bits as a separate add followed by the norm, one launch instead of two.
template <bool RES>
__global__ __launch_bounds__(256) void layer_norm_kernel(float* x, int64_t ldx, const float* __restrict__ res,
                                                         int64_t ldres, float* __restrict__ y, int64_t ldy,
                                                         int64_t rows, int64_t D, const float* __restrict__ gamma,
                                                         const float* __restrict__ beta, float eps) {
    const int64_t r = blockIdx.x;
    if (r >= rows) return;
    float* xr = x + r * ldx;
    if constexpr (RES) {
        const float* rr = res + r * ldres;
        for (int64_t d = threadIdx.x; d < D; d += blockDim.x) xr[d] = xr[d] + rr[d];
    }
    __shared__ float part[8];
    auto block_sum = [&](float v) {
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
        __syncthreads();
        float s = 0.0f;
        for (int w = 0; w < (int)(blockDim.x >> 6); ++w) s += part[w];
        __syncthreads();
        return s;
    };
    float s = 0.0f;
    for (int64_t d = threadIdx.x; d < D; d += blockDim.x) s += xr[d];
    const float mean = block_sum(s) / (float)D;
    float q = 0.0f;
    for (int64_t d = threadIdx.x; d < D; d += blockDim.x) {
        const float c = xr[d] - mean;
        q += c * c;
    }
    const float var = block_sum(q) / (float)D;
    const float inv = 1.0f / sqrtf(var + eps);
    for (int64_t d = threadIdx.x; d < D; d += blockDim.x) {
        float v = (xr[d] - mean) * inv;
        if (gamma) v = v * gamma[d];
        if (beta) v = v + beta[d];
        y[r * ldy + d] = v;
    }
}

// gelu, tanh form: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
__global__ void gelu_tanh_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float v = x[i];
        const float u = 0.7978845608f * (v + 0.044715f * v * v * v);
        y[i] = 0.5f * v * (1.0f + tanhf(u));
    }
}

__global__ void add_kernel(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = a[i] + b[i];
}

// y = a + fl32(b * s): the scaled add of an adapter's update, each operation rounded once
// (the kernel is built without contraction, so no fma fuses them).
__global__ void add_scaled_kernel(const float* __restrict__ a, const float* __restrict__ b, float s, float* __restrict__ y,
                                  int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float t = b[i] * s;
        y[i] = a[i] + t;
    }
}

// y[c][r] = x[r][c] through a 32 x 33 LDS tile (conflict-free transposed reads).
__global__ __launch_bounds__(256) void transpose_kernel(const float* __restrict__ x, int64_t rows, int64_t cols,
                                                        float* __restrict__ y) {
    __shared__ float t[32][33];
    const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
    for (int i = threadIdx.y; i < 32; i += 8) {
        const int64_t r = r0 + i, c = c0 + threadIdx.x;
        if (r < rows && c < cols) t[i][threadIdx.x] = x[r * cols + c];
    }
    __syncthreads();
    for (int i = threadIdx.y; i < 32; i += 8) {
        const int64_t c = c0 + i, r = r0 + threadIdx.x;
        if (r < rows && c < cols) y[c * rows + r] = t[threadIdx.x][i];
    }
}

// qkv [B, n, 3, H, hd] float32 -> q [B, H, n, hd] fp16; k, v appended to the caches
// [B, H, T_max, hd] fp16 at positions pos0 .. pos0 + n - 1.
__global__ void kv_append_kernel(const float* __restrict__ qkv, int64_t B, int64_t n, int64_t H, int64_t hd, int64_t pos0,
                                 const int32_t* __restrict__ d_pos0, int64_t T_max, __half* __restrict__ q,
                                 __half* __restrict__ kc, __half* __restrict__ vc) {
    pos0 = position(pos0, d_pos0, T_max - n);
    const int64_t total = B * n * 3 * H * hd;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        int64_t r = e;
        const int64_t d = r % hd;
        r /= hd;
        const int64_t h = r % H;
        r /= H;
        const int64_t which = r % 3;
        r /= 3;
        const int64_t i = r % n;
        const int64_t b = r / n;
        const __half v = f32_to_f16_rn(qkv[e]);
        if (which == 0) q[((b * H + h) * n + i) * hd + d] = v;
        else (which == 1 ? kc : vc)[((b * H + h) * T_max + pos0 + i) * hd + d] = v;
    }
}

template <int QPB>
__global__ __launch_bounds__(ATT_THREADS) void attention_kernel(const __half* __restrict__ q, const __half* __restrict__ kc,
                                                                const __half* __restrict__ vc, int64_t B, int64_t H,
                                                                int64_t n, int64_t pos0, const int32_t* __restrict__ d_pos0,
                                                                int64_t T_max, float scale, float* __restrict__ out) {
    __shared__ float qs[QPB][ATT_HD];
    __shared__ float p[QPB][ATT_MAX_T];
    __shared__ float rinv[QPB];
    pos0 = position(pos0, d_pos0, min(T_max, (int64_t)ATT_MAX_T) - n);
    const int b = blockIdx.z, h = blockIdx.y, q0 = blockIdx.x * QPB;
    const int nq = (int)min((int64_t)QPB, n - q0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t bh = (int64_t)b * H + h;
    for (int e = tid; e < QPB * ATT_HD; e += ATT_THREADS) {
        const int qi = e / ATT_HD, d = e % ATT_HD;
        qs[qi][d] = qi < nq ? __half2float(q[(bh * n + q0 + qi) * ATT_HD + d]) : 0.0f;
    }
    __syncthreads();
    const int kend = (int)(pos0 + q0 + nq);  // keys 0 .. kend - 1 reach some query of the block
    // scores
    for (int t = tid; t < kend; t += ATT_THREADS) {
        const __half* kr = kc + (bh * T_max + t) * ATT_HD;
        float kv[ATT_HD];
#pragma unroll
        for (int c = 0; c < ATT_HD / 8; ++c) {
            const uint4 w = *reinterpret_cast<const uint4*>(kr + 8 * c);
            const __half* hw = reinterpret_cast<const __half*>(&w);
#pragma unroll
            for (int j = 0; j < 8; ++j) kv[8 * c + j] = __half2float(hw[j]);
        }
#pragma unroll
        for (int qi = 0; qi < QPB; ++qi) {
            float s = 0.0f;
#pragma unroll
            for (int d = 0; d < ATT_HD; ++d) s += qs[qi][d] * kv[d];
            p[qi][t] = (t <= pos0 + q0 + qi) ? s * scale : -INFINITY;
        }
    }
    __syncthreads();
    // softmax weights, rows spread over the waves
    for (int qi = wave; qi < QPB; qi += ATT_THREADS / 64) {
        float m = -INFINITY;
        for (int t = lane; t < kend; t += 64) m = fmaxf(m, p[qi][t]);
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
        float s = 0.0f;
        for (int t = lane; t < kend; t += 64) {
            const float e = expf(p[qi][t] - m);
            p[qi][t] = e;
            s += e;
        }
        for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
        if (lane == 0) rinv[qi] = 1.0f / s;
    }
    __syncthreads();
    // outputs: thread -> (query, dim); lanes run over the 64 dims so V rows load coalesced
    for (int e = tid; e < QPB * ATT_HD; e += ATT_THREADS) {
        const int qi = e / ATT_HD, d = e % ATT_HD;
        if (qi >= nq) continue;
        const int last = (int)(pos0 + q0 + qi);
        float acc = 0.0f;
        const __half* vcol = vc + bh * T_max * ATT_HD + d;
#pragma unroll 8
        for (int t = 0; t <= last; ++t) acc += p[qi][t] * __half2float(vcol[(int64_t)t * ATT_HD]);
        out[(((int64_t)b * n + q0 + qi) * H + h) * ATT_HD + d] = acc * rinv[qi];
    }
}

// Index of the first maximum of each row (numpy argmax; NaN compares as the maximum, as
// numpy's does).  One workgroup per row.
__global__ __launch_bounds__(256) void argmax_kernel(const float* __restrict__ x, int64_t rows, int64_t cols,
                                                     int32_t* __restrict__ idx) {
    const int64_t r = blockIdx.x;
    if (r >= rows) return;
    const float* xr = x + r * cols;
    float bv = -INFINITY;
    int bi = -1;
    for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
        const float v = xr[c];
        const bool better = bi < 0 || (v != v && bv == bv) || v > bv;  // first NaN wins, then the max
        if (better && !(bv != bv)) {
            bv = v;
            bi = (int)c;
        }
    }
    __shared__ float sv[256];
    __shared__ int si[256];
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            const float ov = sv[threadIdx.x + s];
            const int oi = si[threadIdx.x + s];
            const float mv = sv[threadIdx.x];
            const int mi = si[threadIdx.x];
            bool take;
            if (oi < 0) take = false;
            else if (mi < 0) take = true;
            else if (mv != mv) take = (ov != ov) && oi < mi;
            else if (ov != ov) take = true;
            else take = ov > mv || (ov == mv && oi < mi);
            if (take) {
                sv[threadIdx.x] = ov;
                si[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) idx[r] = si[0] < 0 ? 0 : si[0];
}

__global__ void increment_kernel(int32_t* __restrict__ x, int32_t delta) {
    if (threadIdx.x == 0) x[0] += delta;
}

unsigned grid_for(int64_t n) {
    int64_t g = (n + 255) / 256;
    return (unsigned)(g > 65536 ? 65536 : (g < 1 ? 1 : g));
}

}  // namespace
}  // namespace lq

using namespace lq;

extern "C" {

int lq_embedding_sum_f32(const float* d_tok_table, int64_t vocab, const float* d_pos_table, int64_t npos, int64_t D,
                         const int32_t* d_tokens, int64_t rows, int64_t n, int64_t pos0, const int32_t* d_pos0,
                         float* d_out, void* stream) {
    LQ_REQUIRE(vocab > 0 && D > 0 && rows >= 0 && n > 0 && pos0 >= 0 && rows % n == 0 && n <= npos &&
                   (d_pos0 || pos0 + n <= npos),
               "lq_embedding_sum_f32: bad shape");
    if (rows == 0) return LQ_OK;
    LQ_REQUIRE(d_tok_table && d_pos_table && d_tokens && d_out, "lq_embedding_sum_f32: NULL pointer");
    LQ_REQUIRE(rows <= 0x7fffffff, "lq_embedding_sum_f32: too many rows");
    hipLaunchKernelGGL(embedding_sum_kernel, dim3((unsigned)rows), dim3(256), 0, as_stream(stream), d_tok_table,
                       d_pos_table, npos, D, d_tokens, rows, n, pos0, d_pos0, vocab, d_out);
    return launch_status("lq_embedding_sum_f32");
}

int lq_layer_norm_f32(const float* d_x, int64_t ldx, float* d_y, int64_t ldy, int64_t rows, int64_t D,
                      const float* d_gamma, const float* d_beta, float eps, void* stream) {
    LQ_REQUIRE(rows >= 0 && D > 0 && ldx >= D && ldy >= D, "lq_layer_norm_f32: bad shape");
    if (rows == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y, "lq_layer_norm_f32: NULL pointer");
    LQ_REQUIRE(rows <= 0x7fffffff, "lq_layer_norm_f32: too many rows");
    hipLaunchKernelGGL(layer_norm_kernel<false>, dim3((unsigned)rows), dim3(256), 0, as_stream(stream),
                       const_cast<float*>(d_x), ldx, nullptr, 0, d_y, ldy, rows, D, d_gamma, d_beta, eps);
    return launch_status("lq_layer_norm_f32");
}

int lq_add_layer_norm_f32(float* d_x, int64_t ldx, const float* d_res, int64_t ldres, float* d_y, int64_t ldy,
                          int64_t rows, int64_t D, const float* d_gamma, const float* d_beta, float eps,
                          void* stream) {
    LQ_REQUIRE(rows >= 0 && D > 0 && ldx >= D && ldres >= D && ldy >= D, "lq_add_layer_norm_f32: bad shape");
    if (rows == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_res && d_y, "lq_add_layer_norm_f32: NULL pointer");
    LQ_REQUIRE(rows <= 0x7fffffff, "lq_add_layer_norm_f32: too many rows");
    hipLaunchKernelGGL(layer_norm_kernel<true>, dim3((unsigned)rows), dim3(256), 0, as_stream(stream), d_x, ldx,
                       d_res, ldres, d_y, ldy, rows, D, d_gamma, d_beta, eps);
    return launch_status("lq_add_layer_norm_f32");
}

int lq_gelu_tanh_f32(const float* d_x, float* d_y, int64_t n, void* stream) {
    LQ_REQUIRE(n >= 0, "lq_gelu_tanh_f32: n < 0");
    if (n == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y, "lq_gelu_tanh_f32: NULL pointer");
    hipLaunchKernelGGL(gelu_tanh_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), d_x, d_y, n);
    return launch_status("lq_gelu_tanh_f32");
}

int lq_add_f32(const float* d_a, const float* d_b, float* d_y, int64_t n, void* stream) {
    LQ_REQUIRE(n >= 0, "lq_add_f32: n < 0");
    if (n == 0) return LQ_OK;
    LQ_REQUIRE(d_a && d_b && d_y, "lq_add_f32: NULL pointer");
    hipLaunchKernelGGL(add_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), d_a, d_b, d_y, n);
    return launch_status("lq_add_f32");
}

int lq_add_scaled_f32(const float* d_a, const float* d_b, float s, float* d_y, int64_t n, void* stream) {
    LQ_REQUIRE(n >= 0, "lq_add_scaled_f32: n < 0");
    if (n == 0) return LQ_OK;
    LQ_REQUIRE(d_a && d_b && d_y, "lq_add_scaled_f32: NULL pointer");
    hipLaunchKernelGGL(add_scaled_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), d_a, d_b, s, d_y, n);
    return launch_status("lq_add_scaled_f32");
}

int lq_transpose_f32(const float* d_x, int64_t rows, int64_t cols, float* d_y, void* stream) {
    LQ_REQUIRE(rows >= 0 && cols >= 0 && rows < ((int64_t)1 << 36) && cols < ((int64_t)1 << 36),
               "lq_transpose_f32: bad shape");
    if (rows == 0 || cols == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y && d_x != d_y, "lq_transpose_f32: NULL or aliased pointer");
    LQ_REQUIRE((rows + 31) / 32 < 65536, "lq_transpose_f32: too many rows for the grid");
    const dim3 grid((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32));
    hipLaunchKernelGGL(transpose_kernel, grid, dim3(32, 8), 0, as_stream(stream), d_x, rows, cols, d_y);
    return launch_status("lq_transpose_f32");
}

int lq_kv_append_f16(const float* d_qkv, int64_t B, int64_t n, int64_t H, int64_t hd, int64_t pos0,
                     const int32_t* d_pos0, int64_t T_max, void* d_q, void* d_k_cache, void* d_v_cache, void* stream) {
    LQ_REQUIRE(B >= 0 && n >= 0 && H > 0 && hd > 0 && pos0 >= 0 && n <= T_max && (d_pos0 || pos0 + n <= T_max),
               "lq_kv_append_f16: bad shape");
    if (B == 0 || n == 0) return LQ_OK;
    LQ_REQUIRE(d_qkv && d_q && d_k_cache && d_v_cache, "lq_kv_append_f16: NULL pointer");
    const int64_t total = B * n * 3 * H * hd;
    hipLaunchKernelGGL(kv_append_kernel, dim3(grid_for(total)), dim3(256), 0, as_stream(stream), d_qkv, B, n, H, hd, pos0,
                       d_pos0, T_max, (__half*)d_q, (__half*)d_k_cache, (__half*)d_v_cache);
    return launch_status("lq_kv_append_f16");
}

int lq_attention_f16(const void* d_q, const void* d_k_cache, const void* d_v_cache, int64_t B, int64_t H, int64_t n,
                     int64_t hd, int64_t pos0, const int32_t* d_pos0, int64_t T_max, float scale, float* d_out,
                     void* stream) {
    LQ_REQUIRE(B >= 0 && H > 0 && n >= 0 && pos0 >= 0 && n <= T_max && (d_pos0 || pos0 + n <= T_max),
               "lq_attention_f16: bad shape");
    if (hd != ATT_HD) return set_error(LQ_ERR_UNSUPPORTED, "lq_attention_f16: head dim must be 64");
    if ((d_pos0 ? n : pos0 + n) > ATT_MAX_T)
        return set_error(LQ_ERR_UNSUPPORTED, "lq_attention_f16: more than 2048 keys");
    if (B == 0 || n == 0) return LQ_OK;
    LQ_REQUIRE(d_q && d_k_cache && d_v_cache && d_out, "lq_attention_f16: NULL pointer");
    LQ_REQUIRE(B <= 65535 && H <= 65535, "lq_attention_f16: grid too large");
    hipStream_t st = as_stream(stream);
    if (n == 1) {
        hipLaunchKernelGGL((attention_kernel<1>), dim3(1, (unsigned)H, (unsigned)B), dim3(ATT_THREADS), 0, st,
                           (const __half*)d_q, (const __half*)d_k_cache, (const __half*)d_v_cache, B, H, n, pos0,
                           d_pos0, T_max, scale, d_out);
    } else {
        hipLaunchKernelGGL((attention_kernel<8>), dim3((unsigned)((n + 7) / 8), (unsigned)H, (unsigned)B),
                           dim3(ATT_THREADS), 0, st, (const __half*)d_q, (const __half*)d_k_cache,
                           (const __half*)d_v_cache, B, H, n, pos0, d_pos0, T_max, scale, d_out);
    }
    return launch_status("lq_attention_f16");
}

int lq_increment_i32(int32_t* d_x, int32_t delta, void* stream) {
    LQ_REQUIRE(d_x, "lq_increment_i32: NULL pointer");
    hipLaunchKernelGGL(increment_kernel, dim3(1), dim3(64), 0, as_stream(stream), d_x, delta);
    return launch_status("lq_increment_i32");
}

int lq_argmax_f32(const float* d_x, int64_t rows, int64_t cols, int32_t* d_idx, void* stream) {
    LQ_REQUIRE(rows >= 0 && cols > 0 && cols <= 0x7fffffff, "lq_argmax_f32: bad shape");
    if (rows == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_idx, "lq_argmax_f32: NULL pointer");
    LQ_REQUIRE(rows <= 0x7fffffff, "lq_argmax_f32: too many rows");
    hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(256), 0, as_stream(stream), d_x, rows, cols, d_idx);
    return launch_status("lq_argmax_f32");
}

}  // extern "C"
