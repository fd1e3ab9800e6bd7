// lq_glue.hip -- the float kernels a dynamically quantized transformer runs between its int8
// Linears (token + position embedding, layer norm, causal
// attention over an fp16 KV cache, GELU, residual adds, greedy argmax).  They follow Lucid's
// float modules (lucid/nn/modules/normalization.py LayerNorm, nn/functional/attention.py
// scaled_dot_product_attention with is_causal, nn/functional/activation.py gelu tanh form);
// their results are compared with float64 restatements within tolerance (their summation
// order is not knowable from the reference either).
//
// Attention.  Several queries (prefill): flash attention on MFMA, one workgroup per (batch,
// head, 64 queries) streaming 32-key blocks through LDS (attention_mfma_kernel).  One query
// (decode): one workgroup per (batch, head) over the whole key range, scores and weighted V
// rows spread over its 256 threads (attention_decode_kernel), optionally taking the step's
// q / k / v straight from the qkv projection and appending k / v to the caches itself.
// Query i (absolute position pos0 + i) sees keys 0 .. pos0 + i.  KV cache layout
// [B][H][T_max][hd] fp16.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "lq_internal.h"

namespace lq {
namespace {

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

// y = (x - mean) / sqrt(var + eps) [* gamma + beta]: mean and biased variance in float32, one
// wave per row in ln_load / ln_norm's order (the order of every fused norm), four rows per
// workgroup.  RES: the row is first replaced by x + res (the residual add, one rounding per
// element), and the norm runs on the sums: the same bits as a separate add followed by the
// norm, one launch instead of two.  MAXC 0: rows too wide for registers (ln_row_wide).
constexpr int LN_ROWS_PER_WG = 4;
template <int MAXC>
__global__ __launch_bounds__(LN_T * LN_ROWS_PER_WG) void layer_norm_kernel(
    float* x, int64_t ldx, const float* __restrict__ res, int64_t ldres, float* y, int64_t ldy, int64_t rows,
    int64_t D, const float* __restrict__ gamma, const float* __restrict__ beta, float eps) {
    const int64_t r = (int64_t)blockIdx.x * LN_ROWS_PER_WG + (threadIdx.x / LN_T);
    const int t = threadIdx.x % LN_T;
    if (r >= rows) return;  // a whole wave: no barrier follows
    float* xr = x + r * ldx;
    const float* rr = res ? res + r * ldres : nullptr;
    if constexpr (MAXC == 0) {
        ln_row_wide(xr, rr, true, (int)D, t, gamma, beta, eps, y + r * ldy);
    } else {
        float v[4 * MAXC];
        ln_load<MAXC>(xr, rr, xr, true, (int)D, t, v);
        ln_norm<MAXC>(v, true, (int)D, t, gamma, beta, eps, y + r * ldy);
    }
}

// gelu, tanh form: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
__global__ void gelu_tanh_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = gelu_tanh_f32(x[i]);
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

typedef _Float16 h4v __attribute__((ext_vector_type(4)));
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));

// The same copy, eight consecutive head dims per lane (hd % 8 == 0, 16-byte aligned buffers,
// fewer than 2^31 vectors) and 32-bit index arithmetic (the element-wise form's 64-bit
// divisions cost more than its memory traffic).  F32SRC: two 16-byte float loads and the same
// per-element rounding; otherwise qkv is already fp16 (the projection's epilogue rounded it
// the same way) and the lane moves one 16-byte load to one 16-byte store.
template <bool F32SRC>
__global__ __launch_bounds__(256) void kv_append_vec_kernel(const void* __restrict__ qkv, uint32_t rows, uint32_t n,
                                                            uint32_t H, uint32_t hd, int64_t pos0,
                                                            const int32_t* __restrict__ d_pos0, int64_t T_max,
                                                            __half* __restrict__ q, __half* __restrict__ kc,
                                                            __half* __restrict__ vc) {
    pos0 = position(pos0, d_pos0, T_max - n);
    const uint32_t hd8 = hd >> 3, hv = H * hd8, per_row = 3 * hv;
    const uint32_t total = rows * per_row;
    for (uint32_t e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
        h8v o;
        if constexpr (F32SRC) {
            const f4v* src = static_cast<const f4v*>(qkv);
            const f4v a = __builtin_nontemporal_load(&src[2 * (size_t)e]);
            const f4v c = __builtin_nontemporal_load(&src[2 * (size_t)e + 1]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const __half lo = f32_to_f16_rn(a[j]), hi = f32_to_f16_rn(c[j]);
                o[j] = __builtin_bit_cast(_Float16, lo);
                o[j + 4] = __builtin_bit_cast(_Float16, hi);
            }
        } else {
            o = __builtin_nontemporal_load(&static_cast<const h8v*>(qkv)[e]);
        }
        const uint32_t row = e / per_row, w = e - row * per_row;
        const uint32_t which = w / hv, rem = w - which * hv;
        const uint32_t h = rem / hd8, d = (rem - h * hd8) * 8;
        const uint32_t b = row / n, i = row - b * n;
        const int64_t bh = (int64_t)b * H + h;
        __half* dst = which == 0 ? q + (bh * n + i) * hd + d
                                 : (which == 1 ? kc : vc) + (bh * T_max + pos0 + i) * hd + d;
        *reinterpret_cast<h8v*>(dst) = o;
    }
}

// Flash attention over blocks of FA_Q queries (4 waves x 16) on CDNA4 MFMA.  Per block of
// FA_KB keys, staged in LDS (K rows, and V transposed), each wave computes the score tile
// S^T = K Q^T with v_mfma_f32_16x16x32_f16 -- a lane then holds 4 keys (4g + i) of one query
// (l16), which is exactly the A-operand layout of P in O += P V with
// v_mfma_f32_16x16x16_f16, so the weights never leave registers -- and keeps the running
// max / sum of each query (online softmax, float32); the weights enter the PV product as fp16
// hi + lo halves (about 22 significant bits).  O's accumulator lane holds queries
// 4g + i of one dim, so the per-query rescale factors move there by lane shuffles.  Scores,
// exponentials and the products accumulate in float32 over fp16 q / k / v.  Query i sees keys
// 0 .. pos0 + i (causal); every query sees key 0, so the running max is finite after the
// first block.  Keys are staged FA_STAGE at a time (four FA_KB blocks per pair of barriers)
// and the next stage is loaded into registers while this one is computed.  A workgroup of
// eight waves holds two query blocks, i and nqb - 1 - i (waves 0-3 and 4-7), so under the causal
// mask every workgroup scores the same number of key blocks and each SIMD runs one wave of
// each (with one block per workgroup the last blocks' waves did eight times the first's work
// and set the kernel's time).  The weights are exp2 of scores pre-scaled by log2(e)
// (v_exp_f32); the softmax's VALU work, not the MFMAs, bounds this kernel.
constexpr int FA_Q = 64, FA_KB = 32, FA_STAGE = 128, FA_SUB = FA_STAGE / FA_KB;
constexpr int FA_THREADS = 512;  // two query blocks of four waves
constexpr int FA_CPT = FA_STAGE * ATT_HD / 8 / FA_THREADS;  // 16-byte K (and V) chunks per thread per stage
constexpr int FA_KS = 72;   // K row stride in LDS (halves): 144 B keeps 16-byte rows, staggers banks
constexpr int FA_VS = 136;  // V^T row stride (halves)

__device__ __forceinline__ f4v mfma_16x16x32(h8v a, h8v b, f4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4v mfma_16x16x16(h4v a, h4v b, f4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// EXT: also the extrema keys of every value the workgroup stores, one pair per workgroup in
// part[] (grid order), for the dynamic quantize of the output that follows.
template <bool EXT>
__global__ __launch_bounds__(FA_THREADS) void attention_mfma_kernel(const __half* __restrict__ q, const __half* __restrict__ kc,
                                                             const __half* __restrict__ vc, int64_t B, int64_t H,
                                                             int64_t n, int64_t pos0,
                                                             const int32_t* __restrict__ d_pos0, int64_t T_max,
                                                             float scale, float* __restrict__ out,
                                                             int2* __restrict__ part) {
    __shared__ __attribute__((aligned(16))) _Float16 Ks[FA_STAGE * FA_KS];  // [key][dim]
    __shared__ __attribute__((aligned(16))) _Float16 Vt[ATT_HD * FA_VS];     // [dim][key]
    pos0 = position(pos0, d_pos0, T_max - n);
    const int b = blockIdx.z, h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, l16 = lane & 15;
    const int nqb = (int)((n + FA_Q - 1) / FA_Q);
    const int qb_hi = nqb - 1 - (int)blockIdx.x;  // >= blockIdx.x
    const int qb = wave < 4 ? (int)blockIdx.x : qb_hi;
    const bool active = wave < 4 || qb_hi != (int)blockIdx.x;  // an odd count's middle block once
    const int64_t q0 = (int64_t)qb * FA_Q;
    const int64_t bh = (int64_t)b * H + h;
    const int64_t qw = q0 + (wave & 3) * 16;  // this wave's first query
    // B operand of S^T: query qw + l16, dims 8g .. 8g + 7 and 32 + 8g .. 32 + 8g + 7
    const _Float16* qrow = reinterpret_cast<const _Float16*>(q) + (bh * n + min(qw + l16, n - 1)) * ATT_HD;
    const h8v qf0 = *reinterpret_cast<const h8v*>(qrow + 8 * g);
    const h8v qf1 = *reinterpret_cast<const h8v*>(qrow + 32 + 8 * g);
    const int64_t qabs = pos0 + qw + l16;  // position of the query this lane scores
    // keys some query of this wave's block sees (none for an idle wave), and of either block
    const int64_t kend_w = active ? min(pos0 + q0 + FA_Q, pos0 + n) : 0;
    const int64_t kend = min(pos0 + (int64_t)qb_hi * FA_Q + FA_Q, pos0 + n);
    const float sl2 = scale * 1.44269504088896341f;  // scores in log2 units
    float m_run = -INFINITY, l_run = 0.0f;
    f4v o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = f4v{0.f, 0.f, 0.f, 0.f};

    // staging: thread -> keys kk + 64 u of the stage, dims c8 .. c8 + 7
    const int kk = tid >> 3, c8 = (tid & 7) * 8;
    constexpr int KSTEP = FA_THREADS / 8;
    auto fetch = [&](int64_t kb, uint4 (&kv)[FA_CPT], uint4 (&vv)[FA_CPT]) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < FA_CPT; ++u) {
            const int64_t key = kb + kk + KSTEP * u;
            kv[u] = uint4{0u, 0u, 0u, 0u};
            vv[u] = uint4{0u, 0u, 0u, 0u};
            if (key < kend) {
                kv[u] = *reinterpret_cast<const uint4*>(kc + (bh * T_max + key) * ATT_HD + c8);
                vv[u] = *reinterpret_cast<const uint4*>(vc + (bh * T_max + key) * ATT_HD + c8);
            }
        }
    };
    uint4 kv[FA_CPT], vv[FA_CPT];
    fetch(0, kv, vv);
    for (int64_t kb0 = 0; kb0 < kend; kb0 += FA_STAGE) {
#pragma unroll
        for (int u = 0; u < FA_CPT; ++u) {
            const int key = kk + KSTEP * u;
            *reinterpret_cast<uint4*>(Ks + key * FA_KS + c8) = kv[u];
            const _Float16* vh = reinterpret_cast<const _Float16*>(&vv[u]);
#pragma unroll
            for (int j = 0; j < 8; ++j) Vt[(c8 + j) * FA_VS + key] = vh[j];
        }
        __syncthreads();
        if (kb0 + FA_STAGE < kend) fetch(kb0 + FA_STAGE, kv, vv);  // in flight during this stage
        for (int sb = 0; sb < FA_SUB && kb0 + FA_KB * sb < kend_w; ++sb) {
        const int64_t kb = kb0 + FA_KB * sb;
        // S^T tiles: keys kb + 16 t + 4 g + i against query l16
        f4v sc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const _Float16* kr = Ks + (FA_KB * sb + 16 * t + l16) * FA_KS;
            f4v acc = f4v{0.f, 0.f, 0.f, 0.f};
            acc = mfma_16x16x32(*reinterpret_cast<const h8v*>(kr + 8 * g), qf0, acc);
            acc = mfma_16x16x32(*reinterpret_cast<const h8v*>(kr + 32 + 8 * g), qf1, acc);
            sc[t] = acc;
        }
        float mb = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t key = kb + 16 * t + 4 * g + i;
                const float v = (key <= qabs && key < kend_w) ? sc[t][i] * sl2 : -INFINITY;
                sc[t][i] = v;
                mb = fmaxf(mb, v);
            }
        mb = fmaxf(mb, __shfl_xor(mb, 16, 64));
        mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
        const float m_new = fmaxf(m_run, mb);
        const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
        float ps = 0.0f;
        h4v pa[2], pl[2];  // the weights as fp16 hi + lo: ~22 significant bits into the MFMA
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float pv = __builtin_amdgcn_exp2f(sc[t][i] - m_new);
                ps += pv;
                pa[t][i] = (_Float16)pv;
                pl[t][i] = (_Float16)(pv - (float)pa[t][i]);
            }
        ps += __shfl_xor(ps, 16, 64);
        ps += __shfl_xor(ps, 32, 64);
        l_run = l_run * corr + ps;
        m_run = m_new;
        // O rows are queries 4 g + i: their factors live in lanes 4 g + i
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float ci = __shfl(corr, 4 * g + i, 64);
#pragma unroll
            for (int c = 0; c < 4; ++c) o[c][i] *= ci;
        }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const h4v vb =
                    *reinterpret_cast<const h4v*>(Vt + (16 * c + l16) * FA_VS + FA_KB * sb + 16 * t + 4 * g);
                o[c] = mfma_16x16x16(pa[t], vb, o[c]);
                o[c] = mfma_16x16x16(pl[t], vb, o[c]);
            }
        }
        __syncthreads();
    }
    int32_t kmin = KEY_POS_INF, kmax = KEY_NEG_INF;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float li = __shfl(l_run, 4 * g + i, 64);
        const int64_t qi = qw + 4 * g + i;
        if (active && qi < n) {
            float* orow = out + (((int64_t)b * n + qi) * H + h) * ATT_HD + l16;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float v = o[c][i] / li;
                orow[16 * c] = v;
                if constexpr (EXT) key_accum(kmin, kmax, v);
            }
        }
    }
    if constexpr (EXT) {
        __shared__ int32_t smin[FA_THREADS / 64], smax[FA_THREADS / 64];
        kmin = wave_min(kmin);
        kmax = wave_max(kmax);
        if (lane == 0) {
            smin[wave] = kmin;
            smax[wave] = kmax;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < FA_THREADS / 64; ++w) {
                kmin = min(kmin, smin[w]);
                kmax = max(kmax, smax[w]);
            }
            part[((int64_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x] = make_int2(kmin, kmax);
        }
    }
}

// One query per (batch, head) -- the decode step -- over up to ATT_MAX_T keys: DEC_THREADS
// threads score keys t, t + DEC_THREADS, ... (fp32 dot products of fp16 rows, in dim order),
// the softmax runs over an LDS table, then thread (key slot ks, dim chunk dc) accumulates
// p[t] V[t][8 dc .. 8 dc + 7] over keys t = ks, ks + DEC_SLOTS, ... (16-byte row loads,
// several in flight), and the key slots' partial vectors are added in slot order.  FUSED: the step's
// q, k, v come as float32 from the qkv projection [B][3][H][hd]; k and v are rounded to fp16
// into the caches at the position first (kv_append_kernel's rounding), q into LDS.
constexpr int DEC_THREADS = 1024, DEC_SLOTS = DEC_THREADS / 8;

template <bool FUSED>
__global__ __launch_bounds__(DEC_THREADS) void attention_decode_kernel(const void* __restrict__ qsrc,
                                                                       __half* __restrict__ kc,
                                                                       __half* __restrict__ vc, int64_t B,
                                                                       int64_t H, int64_t pos0,
                                                                       const int32_t* __restrict__ d_pos0,
                                                                       int64_t T_max, float scale,
                                                                       float* __restrict__ out) {
    __shared__ float qs[ATT_HD];
    __shared__ float p[ATT_MAX_T];
    __shared__ float red[DEC_THREADS / 64];
    __shared__ float part[DEC_SLOTS][ATT_HD + 1];
    pos0 = position(pos0, d_pos0, min(T_max, (int64_t)ATT_MAX_T) - 1);
    const int b = blockIdx.y, h = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t bh = (int64_t)b * H + h;
    if (tid < ATT_HD) {
        if constexpr (FUSED) {
            const float* qkv = static_cast<const float*>(qsrc) + (int64_t)b * 3 * H * ATT_HD + (int64_t)h * ATT_HD;
            const __half qh = f32_to_f16_rn(qkv[tid]);
            kc[(bh * T_max + pos0) * ATT_HD + tid] = f32_to_f16_rn(qkv[(int64_t)H * ATT_HD + tid]);
            vc[(bh * T_max + pos0) * ATT_HD + tid] = f32_to_f16_rn(qkv[(int64_t)2 * H * ATT_HD + tid]);
            qs[tid] = __half2float(qh);
        } else {
            qs[tid] = __half2float(static_cast<const __half*>(qsrc)[bh * ATT_HD + tid]);
        }
    }
    __syncthreads();
    const int T = (int)pos0 + 1;
    // scores
    for (int t = tid; t < T; t += DEC_THREADS) {
        const __half* kr = kc + (bh * T_max + t) * ATT_HD;
        uint4 w[ATT_HD / 8];
#pragma unroll
        for (int c = 0; c < ATT_HD / 8; ++c) w[c] = *reinterpret_cast<const uint4*>(kr + 8 * c);
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < ATT_HD / 8; ++c) {
            const __half* hw = reinterpret_cast<const __half*>(&w[c]);
#pragma unroll
            for (int j = 0; j < 8; ++j) s += qs[8 * c + j] * __half2float(hw[j]);
        }
        p[t] = s * scale;
    }
    __syncthreads();
    // softmax over the T scores
    float m = -INFINITY;
    for (int t = tid; t < T; t += DEC_THREADS) m = fmaxf(m, p[t]);
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = red[0];
    for (int w = 1; w < DEC_THREADS / 64; ++w) m = fmaxf(m, red[w]);
    __syncthreads();
    float sum = 0.0f;
    for (int t = tid; t < T; t += DEC_THREADS) {
        const float e = expf(p[t] - m);
        p[t] = e;
        sum += e;
    }
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    sum = 0.0f;
    for (int w = 0; w < DEC_THREADS / 64; ++w) sum += red[w];
    const float rinv = 1.0f / sum;
    // weighted V rows: thread (ks, dc) over keys ks, ks + DEC_SLOTS, ...
    const int ks = tid >> 3, dc = tid & 7;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    const __half* vbase = vc + bh * T_max * ATT_HD + 8 * dc;
    int t = ks;
    for (; t + 3 * DEC_SLOTS < T; t += 4 * DEC_SLOTS) {  // four rows in flight
        uint4 w[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
            w[u] = *reinterpret_cast<const uint4*>(vbase + (int64_t)(t + DEC_SLOTS * u) * ATT_HD);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float pu = p[t + DEC_SLOTS * u];
            const __half* hw = reinterpret_cast<const __half*>(&w[u]);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] += pu * __half2float(hw[j]);
        }
    }
    for (; t < T; t += DEC_SLOTS) {
        const uint4 w = *reinterpret_cast<const uint4*>(vbase + (int64_t)t * ATT_HD);
        const float pu = p[t];
        const __half* hw = reinterpret_cast<const __half*>(&w);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += pu * __half2float(hw[j]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) part[ks][8 * dc + j] = acc[j];
    __syncthreads();
    if (tid < ATT_HD) {
        float o = 0.0f;
        for (int k2 = 0; k2 < DEC_SLOTS; ++k2) o += part[k2][tid];
        out[((int64_t)b * H + h) * ATT_HD + tid] = o * rinv;
    }
}

// Index of the first maximum of each row (numpy argmax; NaN compares as the maximum, as
// numpy's does).  One workgroup of 1024 threads per row: each thread scans its float4s
// (several loads in flight) in index order, then the (value, index) pairs meet by wave
// shuffles and LDS under one rule -- NaN over numbers, larger value, lower index on ties --
// so the result does not depend on the combining order.  With `d_pos`, the first workgroup
// also adds `delta` to *d_pos (the decode step's position advance, which nothing in this
// kernel reads).
__device__ __forceinline__ bool argmax_takes(float ov, int oi, float mv, int mi) {
    if (oi < 0) return false;
    if (mi < 0) return true;
    if (mv != mv) return (ov != ov) && oi < mi;
    if (ov != ov) return true;
    return ov > mv || (ov == mv && oi < mi);
}

__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ x, int64_t rows, int64_t cols,
                                                      int32_t* __restrict__ idx, int32_t* __restrict__ d_pos,
                                                      int32_t delta, bool vec) {
    const int64_t r = blockIdx.x;
    if (d_pos && r == 0 && threadIdx.x == 0) d_pos[0] += delta;
    if (r >= rows) return;
    const float* xr = x + r * cols;
    float bv = -INFINITY;
    int bi = -1;
    auto see = [&](float v, int c) {
        if (argmax_takes(v, c, bv, bi)) {
            bv = v;
            bi = c;
        }
    };
    const int64_t nv = vec ? cols / 4 : 0;
    int64_t i = threadIdx.x;
    for (; i + 3 * 1024 < nv; i += 4 * 1024) {
        vf4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = reinterpret_cast<const vf4*>(xr)[i + 1024 * u];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) see(v[u][e], (int)(4 * (i + 1024 * u) + e));
    }
    for (; i < nv; i += 1024) {
        const vf4 v = reinterpret_cast<const vf4*>(xr)[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) see(v[e], (int)(4 * i + e));
    }
    for (int64_t c = 4 * nv + threadIdx.x; c < cols; c += 1024) see(xr[c], (int)c);
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (argmax_takes(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    __shared__ float sv[16];
    __shared__ int si[16];
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; ++w)
            if (argmax_takes(sv[w], si[w], bv, bi)) {
                bv = sv[w];
                bi = si[w];
            }
        idx[r] = bi < 0 ? 0 : bi;
    }
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

static int launch_layer_norm(float* x, int64_t ldx, const float* res, int64_t ldres, float* y, int64_t ldy,
                             int64_t rows, int64_t D, const float* gamma, const float* beta, float eps,
                             hipStream_t st) {
    const dim3 grid((unsigned)((rows + LN_ROWS_PER_WG - 1) / LN_ROWS_PER_WG)), block(LN_T * LN_ROWS_PER_WG);
    auto go = [&](auto c) {
        hipLaunchKernelGGL((layer_norm_kernel<decltype(c)::value>), grid, block, 0, st, x, ldx, res, ldres, y, ldy,
                           rows, D, gamma, beta, eps);
    };
    if (D <= 4 * LN_T) go(std::integral_constant<int, 1>{});
    else if (D <= 8 * LN_T) go(std::integral_constant<int, 2>{});
    else if (D <= 16 * LN_T) go(std::integral_constant<int, 4>{});
    else if (D <= 32 * LN_T) go(std::integral_constant<int, 8>{});
    else go(std::integral_constant<int, 0>{});
    return LQ_OK;
}

int lq_layer_norm_f32(const float* d_x, int64_t ldx, float* d_y, int64_t ldy, int64_t rows, int64_t D,
                      const float* d_gamma, const float* d_beta, float eps, void* stream) {
    LQ_REQUIRE(rows >= 0 && D > 0 && D < ((int64_t)1 << 30) && ldx >= D && ldy >= D, "lq_layer_norm_f32: bad shape");
    if (rows == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y, "lq_layer_norm_f32: NULL pointer");
    LQ_REQUIRE(rows <= 0x7fffffff, "lq_layer_norm_f32: too many rows");
    launch_layer_norm(const_cast<float*>(d_x), ldx, nullptr, 0, d_y, ldy, rows, D, d_gamma, d_beta, eps,
                      as_stream(stream));
    return launch_status("lq_layer_norm_f32");
}

int lq_add_layer_norm_f32(float* d_x, int64_t ldx, const float* d_res, int64_t ldres, float* d_y, int64_t ldy,
                          int64_t rows, int64_t D, const float* d_gamma, const float* d_beta, float eps,
                          void* stream) {
    LQ_REQUIRE(rows >= 0 && D > 0 && D < ((int64_t)1 << 30) && ldx >= D && ldres >= D && ldy >= D,
               "lq_add_layer_norm_f32: bad shape");
    if (rows == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_res && d_y, "lq_add_layer_norm_f32: NULL pointer");
    LQ_REQUIRE(rows <= 0x7fffffff, "lq_add_layer_norm_f32: too many rows");
    launch_layer_norm(d_x, ldx, d_res, ldres, d_y, ldy, rows, D, d_gamma, d_beta, eps, as_stream(stream));
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
    const bool vec = hd % 8 == 0 && total / 8 < ((int64_t)1 << 31) && ((uintptr_t)d_qkv & 15) == 0 &&
                     ((uintptr_t)d_q & 15) == 0 && ((uintptr_t)d_k_cache & 15) == 0 &&
                     ((uintptr_t)d_v_cache & 15) == 0;
    if (vec) {
        hipLaunchKernelGGL(kv_append_vec_kernel<true>, dim3(grid_for(total / 8)), dim3(256), 0, as_stream(stream), d_qkv,
                           (uint32_t)(B * n), (uint32_t)n, (uint32_t)H, (uint32_t)hd, pos0, d_pos0, T_max,
                           (__half*)d_q, (__half*)d_k_cache, (__half*)d_v_cache);
        return launch_status("lq_kv_append_f16");
    }
    hipLaunchKernelGGL(kv_append_kernel, dim3(grid_for(total)), dim3(256), 0, as_stream(stream), d_qkv, B, n, H, hd, pos0,
                       d_pos0, T_max, (__half*)d_q, (__half*)d_k_cache, (__half*)d_v_cache);
    return launch_status("lq_kv_append_f16");
}

int lq_kv_append_h16(const void* d_qkv, int64_t B, int64_t n, int64_t H, int64_t hd, int64_t pos0,
                     const int32_t* d_pos0, int64_t T_max, void* d_q, void* d_k_cache, void* d_v_cache, void* stream) {
    LQ_REQUIRE(B >= 0 && n >= 0 && H > 0 && hd > 0 && pos0 >= 0 && n <= T_max && (d_pos0 || pos0 + n <= T_max),
               "lq_kv_append_h16: bad shape");
    if (B == 0 || n == 0) return LQ_OK;
    LQ_REQUIRE(d_qkv && d_q && d_k_cache && d_v_cache, "lq_kv_append_h16: NULL pointer");
    const int64_t total = B * n * 3 * H * hd;
    LQ_REQUIRE(hd % 8 == 0 && total / 8 < ((int64_t)1 << 31) &&
                   ((reinterpret_cast<uintptr_t>(d_qkv) | reinterpret_cast<uintptr_t>(d_q) |
                     reinterpret_cast<uintptr_t>(d_k_cache) | reinterpret_cast<uintptr_t>(d_v_cache)) & 15) == 0,
               "lq_kv_append_h16: hd must be a multiple of 8 and the buffers 16-byte aligned");
    hipLaunchKernelGGL(kv_append_vec_kernel<false>, dim3(grid_for(total / 8)), dim3(256), 0, as_stream(stream), d_qkv,
                       (uint32_t)(B * n), (uint32_t)n, (uint32_t)H, (uint32_t)hd, pos0, d_pos0, T_max, (__half*)d_q,
                       (__half*)d_k_cache, (__half*)d_v_cache);
    return launch_status("lq_kv_append_h16");
}

int lq_attention_f16(const void* d_q, const void* d_k_cache, const void* d_v_cache, int64_t B, int64_t H, int64_t n,
                     int64_t hd, int64_t pos0, const int32_t* d_pos0, int64_t T_max, float scale, float* d_out,
                     void* stream) {
    LQ_REQUIRE(B >= 0 && H > 0 && n >= 0 && pos0 >= 0 && n <= T_max && (d_pos0 || pos0 + n <= T_max),
               "lq_attention_f16: bad shape");
    if (hd != ATT_HD) return set_error(LQ_ERR_UNSUPPORTED, "lq_attention_f16: head dim must be 64");
    if (n == 1 && (d_pos0 ? min(T_max, (int64_t)ATT_MAX_T + 1) : pos0 + 1) > ATT_MAX_T)
        return set_error(LQ_ERR_UNSUPPORTED, "lq_attention_f16: a single query over more than 2048 keys");
    if (B == 0 || n == 0) return LQ_OK;
    LQ_REQUIRE(d_q && d_k_cache && d_v_cache && d_out, "lq_attention_f16: NULL pointer");
    LQ_REQUIRE(B <= 65535 && H <= 65535, "lq_attention_f16: grid too large");
    hipStream_t st = as_stream(stream);
    if (n == 1) {
        hipLaunchKernelGGL((attention_decode_kernel<false>), dim3((unsigned)H, (unsigned)B), dim3(DEC_THREADS), 0, st,
                           d_q, (__half*)d_k_cache, (__half*)d_v_cache, B, H, pos0, d_pos0, T_max, scale, d_out);
    } else {
        const int64_t nqb = (n + FA_Q - 1) / FA_Q;
        hipLaunchKernelGGL(attention_mfma_kernel<false>, dim3((unsigned)((nqb + 1) / 2), (unsigned)H, (unsigned)B),
                           dim3(FA_THREADS), 0, st, (const __half*)d_q, (const __half*)d_k_cache, (const __half*)d_v_cache,
                           B, H, n, pos0, d_pos0, T_max, scale, d_out, nullptr);
    }
    return launch_status("lq_attention_f16");
}

static int64_t attention_ext_parts(int64_t B, int64_t H, int64_t n) {
    return ((n + FA_Q - 1) / FA_Q + 1) / 2 * H * B;
}

size_t lq_attention_dynamic_quantize_workspace_size(int64_t B, int64_t H, int64_t n, int64_t hd) {
    if (B <= 0 || H <= 0 || n <= 0 || hd <= 0) return 0;
    const size_t parts = sizeof(int2) * (size_t)attention_ext_parts(B, H, n);
    const size_t dq = lq_dynamic_quantize_workspace_size(B * n * H * hd);
    return parts > dq ? parts : dq;
}

int lq_attention_dynamic_quantize_f16(const void* d_q, const void* d_k_cache, const void* d_v_cache, int64_t B,
                                      int64_t H, int64_t n, int64_t hd, int64_t pos0, const int32_t* d_pos0,
                                      int64_t T_max, float scale, float* d_out, int q_dtype, int qmin, int qmax,
                                      float eps, float* d_qparams, void* d_codes, void* d_workspace,
                                      size_t workspace_bytes, void* stream) {
    const char* fn = "lq_attention_dynamic_quantize_f16";
    LQ_REQUIRE(d_qparams && d_codes && qmax > qmin, std::string(fn) + ": NULL output or qmax <= qmin");
    LQ_REQUIRE(workspace_bytes >= lq_attention_dynamic_quantize_workspace_size(B, H, n, hd) && d_workspace,
               std::string(fn) + ": workspace too small");
    const int64_t total = B * n * H * hd;
    const int64_t parts = attention_ext_parts(B, H, n);
    if (n > 1 && hd == ATT_HD && total > 16384 && parts <= DYN_PARTS_MAX &&
        dyn_parts_ok(q_dtype, d_out, d_codes, total, (int)parts)) {
        LQ_REQUIRE(B >= 0 && H > 0 && pos0 >= 0 && n <= T_max && (d_pos0 || pos0 + n <= T_max) && B <= 65535 &&
                       H <= 65535 && d_q && d_k_cache && d_v_cache,
                   std::string(fn) + ": bad shape or NULL input");
        note_path("attention dynamic quantize two-launch");
        const hipStream_t st = as_stream(stream);
        int2* part = static_cast<int2*>(d_workspace);
        const int64_t nqb = (n + FA_Q - 1) / FA_Q;
        hipLaunchKernelGGL(attention_mfma_kernel<true>, dim3((unsigned)((nqb + 1) / 2), (unsigned)H, (unsigned)B),
                           dim3(FA_THREADS), 0, st, (const __half*)d_q, (const __half*)d_k_cache,
                           (const __half*)d_v_cache, B, H, n, pos0, d_pos0, T_max, scale, d_out, part);
        const int rc = launch_status(fn);
        if (rc) return rc;
        return dyn_quantize_parts(d_out, total, q_dtype, qmin, qmax, eps, part, (int)parts, d_qparams, d_codes, st);
    }
    // the separate calls
    int rc = lq_attention_f16(d_q, d_k_cache, d_v_cache, B, H, n, hd, pos0, d_pos0, T_max, scale, d_out, stream);
    if (rc) return rc;
    return lq_dynamic_quantize_f32(d_out, total, q_dtype, qmin, qmax, eps, d_qparams, d_codes, d_workspace,
                                   workspace_bytes, stream);
}

int lq_kv_append_attention_f16(const float* d_qkv, int64_t B, int64_t H, int64_t hd, int64_t pos0,
                               const int32_t* d_pos0, int64_t T_max, void* d_k_cache, void* d_v_cache, float scale,
                               float* d_out, void* stream) {
    LQ_REQUIRE(B >= 0 && H > 0 && pos0 >= 0 && T_max >= 1 && (d_pos0 || pos0 + 1 <= T_max),
               "lq_kv_append_attention_f16: bad shape");
    if (hd != ATT_HD) return set_error(LQ_ERR_UNSUPPORTED, "lq_kv_append_attention_f16: head dim must be 64");
    if ((d_pos0 ? min(T_max, (int64_t)ATT_MAX_T + 1) : pos0 + 1) > ATT_MAX_T)
        return set_error(LQ_ERR_UNSUPPORTED, "lq_kv_append_attention_f16: more than 2048 keys");
    if (B == 0) return LQ_OK;
    LQ_REQUIRE(d_qkv && d_k_cache && d_v_cache && d_out, "lq_kv_append_attention_f16: NULL pointer");
    LQ_REQUIRE(B <= 65535 && H <= 65535, "lq_kv_append_attention_f16: grid too large");
    hipLaunchKernelGGL((attention_decode_kernel<true>), dim3((unsigned)H, (unsigned)B), dim3(DEC_THREADS), 0,
                       as_stream(stream), d_qkv, (__half*)d_k_cache, (__half*)d_v_cache, B, H, pos0, d_pos0, T_max,
                       scale, d_out);
    return launch_status("lq_kv_append_attention_f16");
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
    const bool vec = aligned16(d_x) && cols % 4 == 0;
    hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(1024), 0, as_stream(stream), d_x, rows, cols, d_idx,
                       nullptr, 0, vec);
    return launch_status("lq_argmax_f32");
}

int lq_argmax_next_f32(const float* d_x, int64_t rows, int64_t cols, int32_t* d_idx, int32_t* d_pos, int32_t delta,
                       void* stream) {
    LQ_REQUIRE(rows >= 1 && cols > 0 && cols <= 0x7fffffff && rows <= 0x7fffffff, "lq_argmax_next_f32: bad shape");
    LQ_REQUIRE(d_x && d_idx && d_pos, "lq_argmax_next_f32: NULL pointer");
    const bool vec = aligned16(d_x) && cols % 4 == 0;
    hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(1024), 0, as_stream(stream), d_x, rows, cols, d_idx,
                       d_pos, delta, vec);
    return launch_status("lq_argmax_next_f32");
}

}  // extern "C"
