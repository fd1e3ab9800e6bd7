// lq_wo.hip -- weight-only quantized GEMV / skinny GEMM on CDNA4 MFMA (v_mfma_f32_16x16x32_f16).
//
// Two weight formats, one kernel:
//  * per-channel int8 weights (the sidecar Linear's weight_int8 [N,K], weight_scale [N],
//    weight_zero_point [N]):  y = s[n] * (sum_k c[n,k] x[m,k] - z[n] sum_k x[m,k]) + bias[n]
//    -- Lucid's dequantize -> F.linear for a float input (lucid/nn/quantized/linear.py:206-210);
//  * group-wise packed 4/8-bit weights (QuantizedLinearMLX layout: uint32 words holding
//    32/bits codes little-end first, scales/biases [N, K/gs]):
//    y = sum_g (s[n,g] sum_{k in g} c[n,k] x[m,k] + b[n,g] sum_{k in g} x[m,k]) + bias[n]
//    -- quantized_matmul with transpose=true (lucid/_C/ops/quantized/QuantizedMatmul.cpp:143-163,
//    formula lucid/quantization/_qgemm.py:167-170).
// The transpose=false product x . w_hat (also the QLoRA input gradient) is a separate float32
// tiled kernel, group_matmul_nt_kernel, below.
//
// Operands.  The codes enter the MFMA as exact fp16 values: a code c of 8 or fewer bits is
// placed under the exponent of 1024 (fp16 1024 + c, by v_perm byte placement or nibble
// masks) and 1024 is subtracted in packed fp16.  A float32 activation enters as two fp16
// terms hi + lo after an exact power-of-two pre-scale chosen per (row, k-block) so that the
// block's max |x| lies in [2^14, 2^15): hi = fl16(x 2^e), lo = fl16(x 2^e - hi), ~22
// significant bits per product, fp32 accumulation, and 2^-e applied to the block's sum.  A
// float16 activation is its own hi term.
//
// Work split.  A workgroup of W waves owns 16 weight rows and one 16-row block of the
// activations; its waves split K into equal runs of k-blocks (32*S k each, S = MFMA steps
// per block) and stream their weight bytes with two blocks in flight.  The W partial sums
// meet in LDS and are added in wave order (deterministic), then the epilogue runs.  No
// cross-workgroup synchronisation.  With a workspace, float32 activations are split into
// their hi / lo halves once per call (wo_xprep_kernel) instead of once per workgroup; the
// products and sums are the same either way.
//
// K order inside a k-block: lane q (= l/16) of every step covers 8 consecutive k of its own
// 8*S-wide quarter, so a block stays inside one weight group (group size 32*S) and a lane's
// weight bytes for the block are one contiguous load.  Nibble pairs of a 4-bit word unpack
// in the order 0,4,1,5,2,6,3,7 and the activation halves follow the same order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "lq_internal.h"

namespace lq {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2v __attribute__((ext_vector_type(2)));

constexpr int WO_MAX_WAVES = 16;
constexpr int WO_RING = 4;  // k-blocks in flight per wave

// Waves per workgroup: 16, or 8 for the group-wise variants whose ring of in-flight chunks
// does not fit the 128 registers per lane of a 16-wave workgroup.
constexpr int wo_max_waves(int S, bool xf32, bool grouped) {
    return (grouped && S * (xf32 ? 2 : 1) >= 4) ? 8 : WO_MAX_WAVES;
}

__device__ __forceinline__ h2 bits_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }

// k offset of half h within a lane's 8-element step for a code width.
template <int BITS>
__device__ __forceinline__ int korder(int h) {
    return BITS == 4 ? ((h & 1) * 4 + (h >> 1)) : h;
}

// Four bytes -> four halves (byte - off) in byte order.
__device__ __forceinline__ void bytes_to_h2(uint32_t w, _Float16 off, h2& a, h2& b) {
    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);
    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);
    const h2 o = {off, off};
    a = bits_h2(p0) - o;
    b = bits_h2(p1) - o;
}

// One MFMA step's 8 codes as fp16: 8-bit from two words (signed codes are xor'ed with
// 0x80 so the byte is c + 128), 4-bit from one word.
template <int BITS, bool SIGNED>
__device__ __forceinline__ h8 unpack_step(const uint32_t* w) {
    if constexpr (BITS == 8) {
        const uint32_t x0 = SIGNED ? (w[0] ^ 0x80808080u) : w[0];
        const uint32_t x1 = SIGNED ? (w[1] ^ 0x80808080u) : w[1];
        const _Float16 off = SIGNED ? (_Float16)1152.0f : (_Float16)1024.0f;
        h2 a, b, c, d;
        bytes_to_h2(x0, off, a, b);
        bytes_to_h2(x1, off, c, d);
        return h8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
    } else {
        const h2 o = {(_Float16)1024.0f, (_Float16)1024.0f};
        h2 r[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) r[s] = bits_h2(((w[0] >> (4 * s)) & 0x000F000Fu) | 0x64006400u) - o;
        return h8{r[0].x, r[0].y, r[1].x, r[1].y, r[2].x, r[2].y, r[3].x, r[3].y};
    }
}

__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Epilogue of one output: the float32 product rounded to the activation's type (hmode, a
// LQ_ROUND_* value), the layer bias rounded to that type and added there, then ReLU --
// Lucid's quantized_matmul returning x's dtype and QuantizedLinearMLX's y + bias.to(y.dtype),
// relu (lucid/nn/quantized/mlx_linear.py:215-222).  A half or bfloat16 sum of two such values
// is exact in float32 before its rounding (24 >= 2 p + 2 bits), so the float32 add then round
// equals the narrow add.  hmode 0 leaves the float32 result as it is.
__device__ __forceinline__ float wo_finish(float v, bool has_bias, float b, int relu, int hmode) {
    if (hmode == LQ_ROUND_NONE) {
        if (has_bias) v = v + b;
    } else {
        v = round_result_to(v, hmode);
        if (has_bias) v = round_result_to(v + round_to(b, hmode), hmode);
    }
    if (relu && v <= 0.0f) v = 0.0f;
    return v;
}

// ------------------------------------------------------------------ kernel

struct WoArgs {
    const void* x;
    int64_t ldx;
    const uint8_t* w;        // weight rows (int8 codes, or packed uint32 words as bytes)
    int64_t ldw_bytes;
    const float* w_scale;    // per-channel [N] or group [N][G]
    const float* w_zp;       // per-channel zero points [N] or null
    const float* g_bias;     // group biases [N][G] or null
    const float* bias;       // layer bias [N] or null
    void* y;
    int64_t ldy;
    int relu;
    int hmode;               // LQ_ROUND_*: the activation's float type (group-wise; see wo_finish)
    int M, N, K;
    int G;                   // groups per row (group-wise)
    int bpw;                 // k-blocks per wave (even; blocks past the last are zero work)
    const vu4* xp;           // pre-split activations (wo_xprep_kernel) or null
    const float2* xm;        // per (row, k-block) {2^-e, block sum} of the pre-split activations
};

// A lane's weight bytes for one k-block: 8*S codes from k = kc.
template <int BITS, int S>
struct WChunk {
    static constexpr int NW = S * BITS / 4;  // 32-bit words
    uint32_t w[NW];
};

// A lane's activations for one k-block: 8*S values of one row from k = kc, raw.
template <int S, bool XF32>
struct XChunk {
    static constexpr int NV = XF32 ? 2 * S : S;  // 16-byte units
    vu4 v[NV];
};

// VEC loads are unconditional vector loads (the number in flight stays static, so the
// compiler's wait counts are exact): weight rows past N are clamped to a valid row (their
// outputs are never stored), activation rows past M to the last row, and a chunk at or past
// K re-reads in-row bytes; the activation values of such lanes are replaced by 0 once
// loaded, and an unpacked code is always a finite fp16, so the product is exactly 0.
// Needs 16-byte aligned rows, K % (8S) == 0, K >= 8S.
// !VEC: predicated scalar loads (unaligned rows or a ragged K).
template <int BITS, int S, bool VEC>
__device__ __forceinline__ void load_w(WChunk<BITS, S>& ch, const uint8_t* row, int kc, int K) {
    constexpr int NW = WChunk<BITS, S>::NW;
    constexpr int nk = 8 * S;
    if constexpr (VEC) {
        const uint8_t* p = row + (int64_t)min(kc, K - nk) * BITS / 8;
        if constexpr (NW == 1) {
            ch.w[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
        } else if constexpr (NW == 2) {
            const u2v v = __builtin_nontemporal_load(reinterpret_cast<const u2v*>(p));
            ch.w[0] = v.x; ch.w[1] = v.y;
        } else {
#pragma unroll
            for (int i = 0; i < NW / 4; ++i) {
                const vu4 v = __builtin_nontemporal_load(reinterpret_cast<const vu4*>(p) + i);
                ch.w[4 * i] = v.x; ch.w[4 * i + 1] = v.y; ch.w[4 * i + 2] = v.z; ch.w[4 * i + 3] = v.w;
            }
        }
    } else {
        const uint8_t* p = row + (int64_t)kc * BITS / 8;
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            uint32_t v = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int k = kc + (i * 4 + b) * 8 / BITS;
                if (k < K) v |= (uint32_t)p[i * 4 + b] << (8 * b);
            }
            ch.w[i] = v;
        }
    }
}

template <int S, bool XF32, bool VEC>
__device__ __forceinline__ void load_x(XChunk<S, XF32>& xc, const void* xrow, bool row_ok, int kc, int K) {
    constexpr int NV = XChunk<S, XF32>::NV;
    constexpr int ES = XF32 ? 4 : 2;  // element bytes
    if constexpr (VEC) {
        // always a valid in-row address; rows past M and chunks past K are zeroed after the
        // wait, in compute (a select here would pull the wait forward)
        const vu4* p = reinterpret_cast<const vu4*>(static_cast<const uint8_t*>(xrow) +
                                                    (int64_t)min(kc, K - 8 * S) * ES);
#pragma unroll
        for (int i = 0; i < NV; ++i) xc.v[i] = p[i];
    } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            uint32_t w4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uint32_t word = 0;
                if constexpr (XF32) {
                    const int k = kc + i * 4 + e;
                    if (row_ok && k < K) word = static_cast<const uint32_t*>(xrow)[k];
                } else {
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const int k = kc + i * 8 + e * 2 + hh;
                        if (row_ok && k < K)
                            word |= (uint32_t)static_cast<const uint16_t*>(xrow)[k] << (16 * hh);
                    }
                }
                w4[e] = word;
            }
            xc.v[i] = vu4{w4[0], w4[1], w4[2], w4[3]};
        }
    }
}

template <int S, bool XF32>
__device__ __forceinline__ float x_at(const XChunk<S, XF32>& xc, int i) {
    if constexpr (XF32) {
        return __uint_as_float(xc.v[i >> 2][i & 3]);
    } else {
        const uint32_t w = xc.v[i >> 3][(i >> 1) & 3];
        return (float)bits_h2(w)[i & 1];
    }
}

// A lane's pre-split activations for one k-block: S steps of (hi, lo) halves, and the
// row's {2^-e, block sum}.
template <int S>
struct PChunk {
    vu4 v[2 * S];
    float2 meta;
};

// The float32 activation split of wo_gemv_kernel done once per call instead of once per
// workgroup: one wave per (16-row tile, k-block), lanes laid out as the GEMV's (q = l / 16
// owns 8 S consecutive k of the block, l % 16 the row).  Same zero fill (rows past M, k past
// K), same max / sum shuffles, same power-of-two pre-scale and hi / lo split in the same
// element order, so the GEMV's products and sums are unchanged.  Layout: block (mt, t) holds
// 2 S slots (hi, lo per step) of 64 lanes' vu4 each, lane-contiguous within a slot (coalesced
// 1 KB loads; a lane-major layout made every load touch 64 separate cache lines); meta
// (mt, t, row).
template <int BITS, int S>
__global__ __launch_bounds__(64) void wo_xprep_kernel(const float* __restrict__ x, int64_t ldx, int M, int K, int TW,
                                                      vu4* __restrict__ xp, float2* __restrict__ xm) {
    constexpr int NX = 8 * S;
    const int t = blockIdx.x, mt = blockIdx.y;
    const int lane = threadIdx.x, q = lane >> 4, l16 = lane & 15;
    const int m = mt * 16 + l16;
    const int kc = t * 32 * S + q * 8 * S;
    float xs[NX];
    float amax = 0.0f, bsum = 0.0f;
#pragma unroll
    for (int i = 0; i < NX; ++i) {
        const int k = kc + i;
        xs[i] = (m < M && k < K) ? x[(int64_t)m * ldx + k] : 0.0f;
        amax = fmaxf(amax, fabsf(xs[i]));
        bsum += xs[i];
    }
    amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
    bsum += __shfl_xor(bsum, 16, 64);
    bsum += __shfl_xor(bsum, 32, 64);
    int e = 0;
    if (amax > 0.0f && amax <= 3.0e38f) e = min(max(14 - ilogbf(amax), -120), 120);
    const float up = ldexpf(1.0f, e);
    // slot i of the block's 2 S slots holds the 64 lanes' 16-byte pieces contiguously, so each
    // GEMV load instruction reads 1 KB of consecutive bytes
    vu4* dst = xp + (int64_t)(mt * TW + t) * 2 * S * 64 + lane;
#pragma unroll
    for (int j = 0; j < S; ++j) {
        h8 hi, lo;
#pragma unroll
        for (int h = 0; h < 8; ++h) {
            const float v = xs[8 * j + korder<BITS>(h)] * up;
            const _Float16 vh = (_Float16)v;
            hi[h] = vh;
            lo[h] = (_Float16)(v - (float)vh);
        }
        dst[(2 * j) * 64] = __builtin_bit_cast(vu4, hi);
        dst[(2 * j + 1) * 64] = __builtin_bit_cast(vu4, lo);
    }
    if (q == 0) xm[(int64_t)(mt * TW + t) * 16 + l16] = make_float2(ldexpf(1.0f, -e), bsum);
}

template <int BITS, bool SIGNED, int S, bool XF32, bool GROUPED, bool VEC, bool PREP = false>
__global__ __launch_bounds__((64 * wo_max_waves(S, XF32, GROUPED))) void wo_gemv_kernel(WoArgs a) {
    constexpr int NW = WChunk<BITS, S>::NW;
    constexpr int NX = 8 * S;
    extern __shared__ __attribute__((aligned(16))) float wo_lds[];
    const int W = blockDim.x >> 6;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int q = lane >> 4, l16 = lane & 15;
    const int n0 = blockIdx.x * 16;
    const int m = blockIdx.y * 16 + l16;  // this lane's activation row / output column
    const int TW = W * a.bpw;             // k-blocks over all waves (padded)

    // LDS: [reduction W x 64 x 4][x sums W x 64][group scales 16 x TW][group biases 16 x TW]
    float* red = wo_lds;
    float* redx = red + W * 256;
    float* sc_lds = redx + W * 64;
    float* bi_lds = sc_lds + 16 * TW;
    if constexpr (GROUPED) {
        for (int i = tid; i < 16 * TW; i += blockDim.x) {
            const int n = min(n0 + i / TW, a.N - 1);
            const int64_t gi = (int64_t)n * a.G + min(i % TW, a.G - 1);
            sc_lds[i] = round_to(a.w_scale[gi], a.hmode);
            bi_lds[i] = a.g_bias ? round_to(a.g_bias[gi], a.hmode) : 0.0f;
        }
        __syncthreads();
    }

    const bool row_ok = m < a.M;
    const void* xrow = static_cast<const uint8_t*>(a.x) + (int64_t)min(m, a.M - 1) * a.ldx * (XF32 ? 4 : 2);
    const uint8_t* wrow = a.w + (int64_t)min(n0 + l16, a.N - 1) * a.ldw_bytes;

    f4 acc = f4{0.f, 0.f, 0.f, 0.f};
    float xtot = 0.0f;

    using XC = std::conditional_t<PREP, PChunk<S>, XChunk<S, XF32>>;
    auto load_block = [&](WChunk<BITS, S>& wc, XC& xc, int t) {
        const int kc = t * 32 * S + q * 8 * S;
        load_w<BITS, S, VEC>(wc, wrow, kc, a.K);
        if constexpr (PREP) {
            const int64_t blk = (int64_t)blockIdx.y * TW + t;
            const vu4* src = a.xp + blk * 2 * S * 64 + lane;
#pragma unroll
            for (int i = 0; i < 2 * S; ++i) xc.v[i] = src[i * 64];
            xc.meta = a.xm[blk * 16 + l16];
        } else {
            load_x<S, XF32, VEC>(xc, xrow, row_ok, kc, a.K);
        }
        // keep the prefetch where it is: the scheduler would otherwise sink these loads to
        // their first use and wait on them at once
        __builtin_amdgcn_sched_barrier(0);
    };
    auto compute_prep = [&](const WChunk<BITS, S>& wc, const PChunk<S>& xc, int t) {
        f4 blk = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < S; ++j) {
            const h8 wa = unpack_step<BITS, SIGNED>(&wc.w[j * NW / S]);
            blk = mfma16(wa, __builtin_bit_cast(h8, xc.v[2 * j]), blk);
            blk = mfma16(wa, __builtin_bit_cast(h8, xc.v[2 * j + 1]), blk);
        }
        const float down = xc.meta.x, bsum = xc.meta.y;
        if constexpr (GROUPED) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int rl = 4 * q + i;
                acc[i] += sc_lds[rl * TW + t] * (blk[i] * down) + bi_lds[rl * TW + t] * bsum;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += blk[i] * down;
            xtot += bsum;
        }
    };
    auto compute_raw = [&](const WChunk<BITS, S>& wc, const XChunk<S, XF32>& xc, int t) {
        // the block's pre-scale for this lane's row, shared by the 4 lanes of the row
        float xs[NX];
        float amax = 0.0f, bsum = 0.0f;
        const bool live = row_ok && t * 32 * S + q * 8 * S < a.K;
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            xs[i] = live ? x_at<S, XF32>(xc, i) : 0.0f;
            amax = fmaxf(amax, fabsf(xs[i]));
            bsum += xs[i];
        }
        amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
        bsum += __shfl_xor(bsum, 16, 64);
        bsum += __shfl_xor(bsum, 32, 64);
        int e = 0;
        if (XF32 && amax > 0.0f && amax <= 3.0e38f) e = min(max(14 - ilogbf(amax), -120), 120);
        const float up = XF32 ? ldexpf(1.0f, e) : 1.0f;
        f4 blk = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < S; ++j) {
            h8 hi, lo;
#pragma unroll
            for (int h = 0; h < 8; ++h) {
                const float v = xs[8 * j + korder<BITS>(h)] * up;
                const _Float16 vh = (_Float16)v;
                hi[h] = vh;
                if constexpr (XF32) lo[h] = (_Float16)(v - (float)vh);
            }
            const h8 wa = unpack_step<BITS, SIGNED>(&wc.w[j * NW / S]);
            blk = mfma16(wa, hi, blk);
            if constexpr (XF32) blk = mfma16(wa, lo, blk);
        }
        const float down = XF32 ? ldexpf(1.0f, -e) : 1.0f;
        if constexpr (GROUPED) {
            const int tw = t;  // block index within the padded run of this workgroup
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int rl = 4 * q + i;
                acc[i] += sc_lds[rl * TW + tw] * (blk[i] * down) + bi_lds[rl * TW + tw] * bsum;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += blk[i] * down;
            xtot += bsum;
        }
    };

    // a ring of WO_RING blocks in flight: bpw is a multiple of WO_RING and the last round is
    // peeled, so every load is unconditional and used, and each block's wait leaves the
    // WO_RING - 1 younger blocks in flight
    // (the predicated scalar loads of !VEC keep one block at a time: their registers would
    // not fit a ring)
    auto compute_block = [&](const WChunk<BITS, S>& wc, const XC& xc, int t) {
        if constexpr (PREP) compute_prep(wc, xc, t);
        else compute_raw(wc, xc, t);
    };
    constexpr int RING = VEC ? WO_RING : 1;
    const int t0 = wave * a.bpw;
    WChunk<BITS, S> wr[RING];
    XC xr[RING];
#pragma unroll
    for (int j = 0; j < RING; ++j) load_block(wr[j], xr[j], t0 + j);
    int g = 0;
    for (; g + RING < a.bpw; g += RING) {
#pragma unroll
        for (int j = 0; j < RING; ++j) {
            compute_block(wr[j], xr[j], t0 + g + j);
            load_block(wr[j], xr[j], t0 + g + RING + j);
        }
    }
#pragma unroll
    for (int j = 0; j < RING; ++j) compute_block(wr[j], xr[j], t0 + g + j);

    // partial sums meet in LDS; each output is summed in wave order
    *reinterpret_cast<f4*>(red + (wave * 64 + lane) * 4) = acc;
    if (!GROUPED && q == 0) redx[wave * 64 + l16] = xtot;
    __syncthreads();
    for (int o = tid; o < 256; o += blockDim.x) {  // W may be as small as 1
        const int ol = o >> 2, oi = o & 3;  // output of lane ol, register oi
        const int on = n0 + 4 * (ol >> 4) + oi;
        const int om = blockIdx.y * 16 + (ol & 15);
        if (on < a.N && om < a.M) {
            float v = 0.0f;
            for (int w = 0; w < W; ++w) v += red[(w * 64 + ol) * 4 + oi];
            if constexpr (!GROUPED) {
                if (a.w_zp) {
                    float xt = 0.0f;
                    for (int w = 0; w < W; ++w) xt += redx[w * 64 + (ol & 15)];
                    v = v - a.w_zp[on] * xt;
                }
                v = a.w_scale[on] * v;
            }
            v = wo_finish(v, a.bias != nullptr, a.bias ? a.bias[on] : 0.0f, a.relu, a.hmode);
            if constexpr (XF32)
                reinterpret_cast<float*>(a.y)[(int64_t)om * a.ldy + on] = v;
            else
                reinterpret_cast<_Float16*>(a.y)[(int64_t)om * a.ldy + on] = (_Float16)v;
        }
    }
}

// ------------------------------------------------- split-K skinny GEMM (M <= 16)
//
// wo_gemv_kernel gives each workgroup 16 weight rows and all of K, so every workgroup reads
// the whole 16-row activation block: at M = 16, K = 4096 that is 256 KB per 64 KB of weight,
// ~6x the weight bytes through L2.  Here a workgroup owns SK_TILES 16-row weight tiles (64
// columns) and one K range of 512: it splits its slice of x into fp16 halves once, into LDS,
// where all its waves read it, so x crosses L2 -> CU once per 64 columns.  Its 16 waves are
// SK_TILES tiles x SK_SUB sub-ranges (each wave a few k-blocks, so the 32 waves of two
// workgroups per CU hide each other's latency); the sub-ranges of a tile are added in order
// in LDS.  With one range (K <= 512) the workgroup runs the epilogue; otherwise it stores the
// range's tile sums and wo_sk_reduce_kernel adds the ranges in range order (a second small
// launch: a last-arriving workgroup fixup through agent-scope memory measured slower) and
// runs the epilogue.  The products and per-block sums are those of wo_gemv_kernel (same
// split, same MFMA steps); only the order in which the block sums are added differs.
constexpr int SK_TILES = 4;
constexpr int SK_SUB = 4;
constexpr int SK_WAVES = SK_TILES * SK_SUB;
constexpr int SK_RANGE_K = 512;  // K per workgroup

template <int S>
constexpr int sk_blocks() { return SK_RANGE_K / (32 * S); }  // k-blocks per range: 16 / S

struct WoSkArgs {
    WoArgs w;            // shapes, operands, epilogue (bpw, xp, xm unused)
    int splits;          // K ranges per column group
    float* part;         // [range][group][SK_TILES][64 lanes][4] tile sums
    float* part_x;       // [range][16] activation row sums over the range
};

template <int BITS, bool SIGNED, int S, bool XF32, bool GROUPED, bool PACKED = false>
__global__ __launch_bounds__(64 * SK_WAVES) void wo_gemv_sk_kernel(WoSkArgs sk) {
    const WoArgs& a = sk.w;
    constexpr int NW = WChunk<BITS, S>::NW;
    constexpr int NX = 8 * S;
    constexpr int KB = sk_blocks<S>();        // k-blocks per range
    constexpr int RB = (KB + SK_SUB - 1) / SK_SUB;  // k-blocks per wave
    constexpr int SL = XF32 ? 2 * S : S;      // 16-byte fragments per lane and k-block
    __shared__ vu4 xs[KB * SL * 64];
    __shared__ float2 xmeta[KB * 16];
    __shared__ f4 red[SK_WAVES * 64];
    __shared__ float redx[SK_SUB * 16];
    __shared__ float gsc[GROUPED ? SK_TILES * 16 * KB : 1], gbi[GROUPED ? SK_TILES * 16 * KB : 1];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = wave % SK_TILES, sub = wave / SK_TILES;
    const int q = lane >> 4, l16 = lane & 15;
    const int cg = blockIdx.x, range = blockIdx.y;
    const int TB = (a.K + 32 * S - 1) / (32 * S);
    const int tb0 = range * KB;
    const int nb = min(TB - tb0, KB);          // >= 1 by the grid
    const int n0 = (cg * SK_TILES + tile) * 16;
    const uint8_t* wrow = a.w + (int64_t)min(n0 + l16, a.N - 1) * a.ldw_bytes;
    const bool row_ok = l16 < a.M;
    const void* xrow = static_cast<const uint8_t*>(a.x) + (int64_t)min(l16, a.M - 1) * a.ldx * (XF32 ? 4 : 2);

    // this wave's k-blocks of the range: sub, sub + SK_SUB, ... (blocks past the range
    // re-read its last one: a static number of loads; their products are not added)
    // x first: vmcnt counts in issue order, so the split below waits for x alone
    const int xt = wave;                       // the k-block of x this wave splits (if < nb)
    XChunk<S, XF32> xc;
    load_x<S, XF32, true>(xc, xrow, row_ok, (tb0 + min(xt, nb - 1)) * 32 * S + q * 8 * S, a.K);
    WChunk<BITS, S> wc[RB];
    if constexpr (PACKED) {
        // MFMA-packed int8 weight (lq_pack_weights_i8): tile (n-tile, 64-k step) is 1 KB in
        // this kernel's lane order, so each wave load is 1 KB of consecutive bytes
        static_assert(BITS == 8 && S == 2, "the packed layout holds 64-k steps of int8 codes");
        const int KS = (a.K + 63) / 64;
        const int ntile = min(n0 / 16, (a.N - 1) / 16);
        const uint8_t* tb = a.w + (int64_t)ntile * KS * 1024 + lane * 16;
#pragma unroll
        for (int j = 0; j < RB; ++j) {
            const vu4 v = __builtin_nontemporal_load(
                reinterpret_cast<const vu4*>(tb + (int64_t)(tb0 + min(sub + SK_SUB * j, nb - 1)) * 1024));
            wc[j].w[0] = v.x; wc[j].w[1] = v.y; wc[j].w[2] = v.z; wc[j].w[3] = v.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < RB; ++j)
            load_w<BITS, S, true>(wc[j], wrow, (tb0 + min(sub + SK_SUB * j, nb - 1)) * 32 * S + q * 8 * S, a.K);
    }
    if constexpr (GROUPED) {
        if (sub == 0)
            for (int i = lane; i < 16 * nb; i += 64) {
                const int r = i / nb, t = i - r * nb;
                const int64_t gi = (int64_t)min(n0 + r, a.N - 1) * a.G + (tb0 + t);
                gsc[(tile * 16 + r) * KB + t] = round_to(a.w_scale[gi], a.hmode);
                gbi[(tile * 16 + r) * KB + t] = a.g_bias ? round_to(a.g_bias[gi], a.hmode) : 0.0f;
            }
    }

    // split one k-block of x (KB <= SK_WAVES): the block's pre-scale per row, hi / lo halves
    // in the lanes' fragment order (as wo_xprep_kernel), {2^-e, block sum} per row
    static_assert(KB <= SK_WAVES, "one k-block of x per wave");
    {
        float xv[NX];
        float amax = 0.0f, bsum = 0.0f;
        const bool live = row_ok && xt < nb && (tb0 + xt) * 32 * S + q * 8 * S < a.K;
#pragma unroll
        for (int e = 0; e < NX; ++e) {
            xv[e] = live ? x_at<S, XF32>(xc, e) : 0.0f;
            amax = fmaxf(amax, fabsf(xv[e]));
            bsum += xv[e];
        }
        amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
        bsum += __shfl_xor(bsum, 16, 64);
        bsum += __shfl_xor(bsum, 32, 64);
        int e2 = 0;
        if (XF32 && amax > 0.0f && amax <= 3.0e38f) e2 = min(max(14 - ilogbf(amax), -120), 120);
        const float up = XF32 ? ldexpf(1.0f, e2) : 1.0f;
        if (xt < nb) {
            vu4* dst = xs + xt * SL * 64 + lane;
#pragma unroll
            for (int j = 0; j < S; ++j) {
                h8 hi, lo;
#pragma unroll
                for (int h = 0; h < 8; ++h) {
                    const float v = xv[8 * j + korder<BITS>(h)] * up;
                    const _Float16 vh = (_Float16)v;
                    hi[h] = vh;
                    if constexpr (XF32) lo[h] = (_Float16)(v - (float)vh);
                }
                if constexpr (XF32) {
                    dst[(2 * j) * 64] = __builtin_bit_cast(vu4, hi);
                    dst[(2 * j + 1) * 64] = __builtin_bit_cast(vu4, lo);
                } else {
                    dst[j * 64] = __builtin_bit_cast(vu4, hi);
                }
            }
            if (q == 0) xmeta[xt * 16 + l16] = make_float2(XF32 ? ldexpf(1.0f, -e2) : 1.0f, bsum);
        }
    }
    __syncthreads();

    f4 acc = f4{0.f, 0.f, 0.f, 0.f};
    float xtot = 0.0f;
#pragma unroll
    for (int j = 0; j < RB; ++j) {
        const int t = sub + SK_SUB * j;
        if (t < nb) {  // wave-uniform; a predicate keeps wc[] in registers
            const vu4* xf = xs + t * SL * 64 + lane;
            const float2 mt = xmeta[t * 16 + l16];
            f4 blk = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < S; ++st) {
                const h8 wa = unpack_step<BITS, SIGNED>(&wc[j].w[st * NW / S]);
                if constexpr (XF32) {
                    blk = mfma16(wa, __builtin_bit_cast(h8, xf[(2 * st) * 64]), blk);
                    blk = mfma16(wa, __builtin_bit_cast(h8, xf[(2 * st + 1) * 64]), blk);
                } else {
                    blk = mfma16(wa, __builtin_bit_cast(h8, xf[st * 64]), blk);
                }
            }
            if constexpr (GROUPED) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = (tile * 16 + 4 * q + i) * KB + t;
                    acc[i] += gsc[r] * (blk[i] * mt.x) + gbi[r] * mt.y;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] += blk[i] * mt.x;
                xtot += mt.y;
            }
        }
    }
    // the sub-ranges of each tile meet in LDS, added in sub-range order
    red[wave * 64 + lane] = acc;
    if (!GROUPED && tile == 0 && q == 0) redx[sub * 16 + l16] = xtot;
    __syncthreads();
    if (sub != 0) return;
    acc = red[tile * 64 + lane];
    xtot = redx[l16];
#pragma unroll
    for (int u = 1; u < SK_SUB; ++u) {
        acc += red[(u * SK_TILES + tile) * 64 + lane];
        if (!GROUPED) xtot += redx[u * 16 + l16];
    }
    if (sk.splits > 1) {
        float* dst = sk.part + (((int64_t)range * gridDim.x + cg) * SK_TILES + tile) * 256 + lane * 4;
        *reinterpret_cast<f4*>(dst) = acc;
        if (!GROUPED && tile == 0 && q == 0 && cg == 0) sk.part_x[range * 16 + l16] = xtot;
        return;
    }
    if (n0 >= a.N || !row_ok) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = n0 + 4 * q + i;
        if (n < a.N) {
            float v = acc[i];
            if constexpr (!GROUPED) {
                if (a.w_zp) v = v - a.w_zp[n] * xtot;
                v = a.w_scale[n] * v;
            }
            v = wo_finish(v, a.bias != nullptr, a.bias ? a.bias[n] : 0.0f, a.relu, a.hmode);
            if constexpr (XF32)
                reinterpret_cast<float*>(a.y)[(int64_t)l16 * a.ldy + n] = v;
            else
                reinterpret_cast<_Float16*>(a.y)[(int64_t)l16 * a.ldy + n] = (_Float16)v;
        }
    }
}

// Adds the K ranges' tile sums in range order and runs the epilogue: one thread per lane
// slot of a tile (4 outputs of one activation row).
template <bool XF32, bool GROUPED>
__global__ __launch_bounds__(256) void wo_sk_reduce_kernel(WoSkArgs sk, int groups) {
    const WoArgs& a = sk.w;
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (group, tile, lane)
    if (g >= (int64_t)groups * SK_TILES * 64) return;
    const int lane = (int)(g & 63), q = lane >> 4, l16 = lane & 15;
    const int64_t gt = g >> 6;  // group * SK_TILES + tile
    const int n0 = (int)(gt * 16);
    if (n0 >= a.N || l16 >= a.M) return;
    // the epilogue's per-column inputs are loaded with the partial sums, not after them
    float wsc[4], wzp[4], wbi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = min(n0 + 4 * q + i, a.N - 1);  // clamped: columns past N are never stored
        wsc[i] = GROUPED ? 1.0f : a.w_scale[n];
        wzp[i] = (!GROUPED && a.w_zp) ? a.w_zp[n] : 0.0f;
        wbi[i] = a.bias ? a.bias[n] : 0.0f;
    }
    f4 acc = f4{0.f, 0.f, 0.f, 0.f};
    float xtot = 0.0f;
    // eight ranges' loads in flight, then their sums in range order
    for (int r0 = 0; r0 < sk.splits; r0 += 8) {
        f4 v[8];
        float xv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int r = min(r0 + u, sk.splits - 1);
            v[u] = *reinterpret_cast<const f4*>(sk.part + ((int64_t)r * groups * SK_TILES + gt) * 256 + lane * 4);
            xv[u] = GROUPED ? 0.0f : sk.part_x[r * 16 + l16];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (r0 + u < sk.splits) {
                acc += v[u];
                if (!GROUPED) xtot += xv[u];
            }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = n0 + 4 * q + i;
        if (n < a.N) {
            float v = acc[i];
            if constexpr (!GROUPED) {
                if (a.w_zp) v = v - wzp[i] * xtot;
                v = wsc[i] * v;
            }
            v = wo_finish(v, a.bias != nullptr, wbi[i], a.relu, a.hmode);
            if constexpr (XF32)
                reinterpret_cast<float*>(a.y)[(int64_t)l16 * a.ldy + n] = v;
            else
                reinterpret_cast<_Float16*>(a.y)[(int64_t)l16 * a.ldy + n] = (_Float16)v;
        }
    }
}

// ------------------------------------------------- one or two activation rows (VALU)
//
// For M <= 2 the MFMA's 16 activation columns are mostly empty and the per-block hi/lo split
// of x would dominate; a classic GEMV is cheaper.  The workgroup stages its (at most two)
// activation rows in LDS as fp32 once; each wave then owns whole weight rows: lane l takes
// the 16-byte chunks l, l + 64, ... of its row, issues all of them at once (J chunks in flight,
// J a template step), converts each code with one instruction (v_cvt_f32_i32 / ubyte with a
// byte select) and accumulates in fp32 with FMA.  A 64-lane shuffle reduction finishes each
// row.  The LDS copy of x is swizzled (16-byte slot f of a 256-byte row stored at
// f ^ ... rotated by f >> 4) so the 64 lanes' float4 reads of their chunks are conflict-free.
// One activation row, per-channel weights, K <= 256 * 16 codes (wv_persistent): the grid is
// persistent (at most one workgroup per CU): wave w of workgroup b takes rows gw, gw + S, ...
// (gw = b * waves + w, S = all waves of the grid), staging x once per workgroup, and loads the
// next row's chunks before it reduces the current one.  Each row's arithmetic is the same as
// with one row per wave (same bits).  The other forms keep one row per wave: a second row's
// chunks in flight would not fit their registers.

struct WvArgs {
    const void* x;
    int64_t ldx;
    const uint8_t* w;
    int64_t ldw_bytes;
    const float* w_scale;    // per-channel [N] or group [N][G]
    const float* w_zp;       // per-channel zero points [N] or null
    const float* g_bias;     // group biases [N][G] or null
    const float* bias;       // layer bias [N] or null
    void* y;
    int64_t ldy;
    int relu;
    int hmode;               // LQ_ROUND_* (see wo_finish)
    int M, N, K;
    int G, gs;
    int NC;                  // 16-byte chunks per weight row
    int Kpad;                // staged activation length (J * 64 chunks of codes)
    int xvec;                // activation rows allow 4-element vector loads
};

__device__ __forceinline__ int wv_slot(int k) {
    // float index k -> swizzled float index: 16-byte slot f = k / 4 rotated within its
    // 256-byte LDS row by f >> 4
    const int f = k >> 2;
    return (((f & ~15) | ((f + (f >> 4)) & 15)) << 2) | (k & 3);
}

// Staged activation index 4 * i -> (row m, element k) of the [MX][Kpad] copy, MX <= 2: a
// compare instead of an integer division by the runtime Kpad.
template <int MX>
__device__ __forceinline__ int wv_row(int e4, int Kpad) {
    static_assert(MX == 1 || MX == 2, "one or two activation rows");
    return MX == 2 && e4 >= Kpad ? 1 : 0;
}

__device__ __forceinline__ uint32_t opaque_and(uint32_t v, uint32_t m) {
    uint32_t r;
    __asm__("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(v), "v"(m));
    return r;
}

constexpr bool wv_persistent(bool grouped, int mx, int j) { return !grouped && mx == 1 && j <= 4; }

template <int BITS, bool SIGNED, bool GROUPED, int MX, bool XF32, int J, int HM = LQ_ROUND_NONE>
__global__ __launch_bounds__(1024) void wo_gemv_valu_kernel(WvArgs a) {
    // HM: the group scales' rounding (a.hmode as a constant, so the default costs nothing)
    constexpr int CK = 16 * 8 / BITS;  // codes per 16-byte chunk
    extern __shared__ __attribute__((aligned(16))) float wv_lds[];
    float* xs = wv_lds;                                   // [MX][Kpad], swizzled
    float* gsum = xs + MX * a.Kpad;                       // [MX][G] (group-wise) or [MX] totals
    constexpr bool PF = wv_persistent(GROUPED, MX, J);  // rows in a loop, the next one prefetched
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int waves = blockDim.x >> 6;
    const int gw = blockIdx.x * waves + wave;  // this wave's first row
    const int wstride = gridDim.x * waves;

    // every chunk load of a row at once (clamped to the row; chunks past the row meet zero x)
    auto load_row = [&](int n, vu4* w, float* sgv, float* bgv) {
        const uint8_t* row = a.w + (int64_t)n * a.ldw_bytes;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int c = min(lane + 64 * j, a.NC - 1);
            w[j] = __builtin_nontemporal_load(reinterpret_cast<const vu4*>(row) + c);
            if constexpr (GROUPED) {
                const int64_t gi = (int64_t)n * a.G + min((lane + 64 * j) * CK / a.gs, a.G - 1);
                sgv[j] = a.w_scale[gi];  // rounded to x's type where used: a rounding here would
                bgv[j] = a.g_bias ? a.g_bias[gi] : 0.0f;  // wait for the prefetched row's loads
            }
        }
    };
    // the first row's loads go out before the activation staging so the two latencies overlap
    vu4 wc[J];
    float sg[GROUPED ? J : 1], bg[GROUPED ? J : 1];
    load_row(min(gw, a.N - 1), wc, sg, bg);
    __builtin_amdgcn_sched_barrier(0);

    // Activation staging in groups of four consecutive k (one 16-byte LDS slot; Kpad is a
    // multiple of 4), up to XU groups per thread with every load issued before any LDS store,
    // so the staging costs one L2 round trip per XU * blockDim.x groups instead of one per
    // element.  Vector loads when the rows allow them (a.xvec), element loads otherwise.
    constexpr int XU = 4;
    const int nq = MX * a.Kpad / 4;
    for (int base = 0; base < nq; base += XU * (int)blockDim.x) {
        vf4 xv4[XU];
#pragma unroll
        for (int u = 0; u < XU; ++u) {
            const int i = base + u * (int)blockDim.x + tid;
            const int m = wv_row<MX>(4 * i, a.Kpad), k = (4 * i) - m * a.Kpad;
            vf4 v = vf4{0.0f, 0.0f, 0.0f, 0.0f};
            if (i < nq && m < a.M && k < a.K) {
                const int64_t o = (int64_t)m * a.ldx + k;
                if (a.xvec && k + 4 <= a.K) {
                    if constexpr (XF32) {
                        v = *reinterpret_cast<const vf4*>(static_cast<const float*>(a.x) + o);
                    } else {
                        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                        const h4 h = *reinterpret_cast<const h4*>(static_cast<const _Float16*>(a.x) + o);
                        v = vf4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (k + e < a.K) {
                            if constexpr (XF32) v[e] = static_cast<const float*>(a.x)[o + e];
                            else v[e] = (float)static_cast<const _Float16*>(a.x)[o + e];
                        }
                    }
                }
            }
            xv4[u] = v;
        }
#pragma unroll
        for (int u = 0; u < XU; ++u) {
            const int i = base + u * (int)blockDim.x + tid;
            if (i < nq) {
                const int m = wv_row<MX>(4 * i, a.Kpad), k = (4 * i) - m * a.Kpad;
                *reinterpret_cast<vf4*>(xs + m * a.Kpad + wv_slot(k)) = xv4[u];
            }
        }
    }
    __syncthreads();
    // x sums: per group (group-wise) or per row (zero points), from float4 partials reduced
    // across the lanes of a group by shuffles, then in fixed order across waves
    if (GROUPED || a.w_zp) {
        const int span = GROUPED ? a.gs : a.Kpad;  // elements summed into one value
        const int per = span / 4;                  // float4 partials per value
        float* wsum = gsum + (GROUPED ? MX * a.G : MX);  // [waves][MX] (zero-point totals)
        for (int i0 = 0; i0 < MX * a.Kpad / 4; i0 += blockDim.x) {
            const int i = i0 + tid;
            float v = 0.0f;
            if (i < MX * a.Kpad / 4) {
                const int m = wv_row<MX>(4 * i, a.Kpad), k = (4 * i) - m * a.Kpad;
                const vf4 q = *reinterpret_cast<const vf4*>(xs + m * a.Kpad + wv_slot(k));
                v = (q[0] + q[1]) + (q[2] + q[3]);
            }
            if (GROUPED) {
                // per <= 32 lanes of one group are consecutive threads of one wave
#pragma unroll
                for (int off = 1; off < 64; off <<= 1)
                    if (off < per) v += __shfl_xor(v, off, 64);
                if (i < MX * a.Kpad / 4 && (i % per) == 0) {
                    const int m = wv_row<MX>(4 * i, a.Kpad), k = (4 * i) - m * a.Kpad;
                    if (k < a.K) gsum[m * a.G + k / a.gs] = v;  // Kpad is a multiple of gs
                }
            } else {
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
                // a wave's 64 partials lie in one row (Kpad is a multiple of 256)
                if (lane == 0 && i0 + wave * 64 < MX * a.Kpad / 4) {
                    const int m = wv_row<MX>(4 * (i0 + wave * 64), a.Kpad);
                    const int slot = (i0 / (int)blockDim.x) * waves + wave;
                    wsum[slot * MX + m] = v;  // distinct slot per (pass, wave); zero for other rows below
                }
            }
        }
        if (!GROUPED) {
            __syncthreads();
            if (tid < MX) {
                const int passes = (MX * a.Kpad / 4 + blockDim.x - 1) / blockDim.x;
                float t = 0.0f;
                for (int sidx = 0; sidx < passes * waves; ++sidx) {
                    const int i = (sidx / waves) * blockDim.x + (sidx % waves) * 64;
                    if (i < MX * a.Kpad / 4 && wv_row<MX>(4 * i, a.Kpad) == tid) t += wsum[sidx * MX + tid];
                }
                gsum[tid] = t;
            }
        }
        __syncthreads();
    }
    if (gw >= a.N) return;

    for (int n = gw; n < a.N; n += wstride) {
        const int nn = n + wstride;
        const bool more = PF && nn < a.N;  // wave-uniform
        vu4 wn[PF ? J : 1];
        float sgn[PF && GROUPED ? J : 1], bgn[PF && GROUPED ? J : 1];
        if (more) load_row(nn, wn, sgn, bgn);
        float acc[MX];
#pragma unroll
        for (int m = 0; m < MX; ++m) acc[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int c = lane + 64 * j;
            const int k0 = c * CK;
            float p[MX];
#pragma unroll
            for (int m = 0; m < MX; ++m) p[m] = 0.0f;
#pragma unroll
            for (int wi = 0; wi < 4; ++wi) {
                const uint32_t wd = wc[j][wi];
                float code[32 / BITS];
                if constexpr (BITS == 8) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        code[e] = SIGNED ? (float)(signed char)(wd >> (8 * e)) : (float)((wd >> (8 * e)) & 0xFFu);
                } else {
                    const uint32_t lo = opaque_and(wd, 0x0F0F0F0Fu);
                    const uint32_t hi = opaque_and(wd >> 4, 0x0F0F0F0Fu);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        code[2 * e] = (float)((lo >> (8 * e)) & 0xFFu);
                        code[2 * e + 1] = (float)((hi >> (8 * e)) & 0xFFu);
                    }
                }
                const int kw = k0 + wi * (32 / BITS);
#pragma unroll
                for (int m = 0; m < MX; ++m) {
#pragma unroll
                    for (int f = 0; f < 32 / BITS; f += 4) {
                        const vf4 xv = *reinterpret_cast<const vf4*>(xs + m * a.Kpad + wv_slot(kw + f));
#pragma unroll
                        for (int e = 0; e < 4; ++e) p[m] = fmaf(code[f + e], xv[e], p[m]);
                    }
                }
            }
            if constexpr (GROUPED) {
                const bool first = c < a.NC && (k0 % a.gs) == 0;
                const int g = min(k0 / a.gs, a.G - 1);
#pragma unroll
                for (int m = 0; m < MX; ++m) {
                    acc[m] = fmaf(round_to(sg[j], HM), p[m], acc[m]);
                    if (first) acc[m] = fmaf(round_to(bg[j], HM), gsum[m * a.G + g], acc[m]);
                }
            } else {
#pragma unroll
                for (int m = 0; m < MX; ++m) acc[m] += p[m];
            }
        }
#pragma unroll
        for (int m = 0; m < MX; ++m) {
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) acc[m] += __shfl_xor(acc[m], off, 64);
        }
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < MX; ++m) {
                if (m >= a.M) break;
                float v = acc[m];
                if constexpr (!GROUPED) {
                    if (a.w_zp) v = v - a.w_zp[n] * gsum[m];
                    v = a.w_scale[n] * v;
                }
                v = wo_finish(v, a.bias != nullptr, a.bias ? a.bias[n] : 0.0f, a.relu, a.hmode);
                if constexpr (XF32)
                    reinterpret_cast<float*>(a.y)[(int64_t)m * a.ldy + n] = v;
                else
                    reinterpret_cast<_Float16*>(a.y)[(int64_t)m * a.ldy + n] = (_Float16)v;
            }
        }
        if constexpr (!PF) break;  // one row per wave (the grid covers every row)
        if (more) {
#pragma unroll
            for (int j = 0; j < J; ++j) {
                wc[j] = wn[j];
                if constexpr (GROUPED) sg[j] = sgn[j], bg[j] = bgn[j];
            }
        }
    }  // rows of this wave
}

// ------------------------------------------------- group-wise quantize / dequantize

// One thread per (row, group): s = (max - min) / (2^bits - 1), b = min,
// c = clip(rne((w - b) / s), 0, 2^bits - 1) (formula lucid/quantization/_qgemm.py:84-97; a
// group with max == min, or a NaN range, keeps s as computed and codes 0).  Codes are packed
// 32/bits per uint32, little-end first.
template <int BITS>
__global__ __launch_bounds__(256) void group_quantize_kernel(const float* __restrict__ w, int64_t N, int64_t K,
                                                             int gs, uint32_t* __restrict__ packed,
                                                             float* __restrict__ scales,
                                                             float* __restrict__ biases) {
    const int64_t G = K / gs;
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= N * G) return;
    const int64_t n = id / G, g = id - n * G;
    const float* p = w + n * K + g * gs;
    float mn = __int_as_float(0x7f800000), mx = -__int_as_float(0x7f800000);
    for (int i = 0; i < gs; i += 4) {
        const vf4 v = *reinterpret_cast<const vf4*>(p + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            mn = extreme_min(mn, v[e]);
            mx = extreme_max(mx, v[e]);
        }
    }
    constexpr uint32_t L = (1u << BITS) - 1u;
    constexpr int PER = 32 / BITS;
    const float s = (mx - mn) / (float)L;
    scales[id] = s;
    biases[id] = mn;
    uint32_t* out = packed + (n * K + g * gs) / PER;
    for (int i = 0; i < gs; i += PER) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            uint32_t c = 0;
            if (s > 0.0f) {
                const float d = p[i + e] - mn;
                const float t = d / s;
                c = (uint32_t)satcast<int32_t>(clip_tie(rne(t), 0.0f, (float)L, true, false), 0.0f,
                                               (float)L, 0, (int)L);
            }
            word |= c << (e * BITS);
        }
        out[i / PER] = word;
    }
}

// w_hat = fl32(fl32(c * s) + b) (lucid/quantization/_qgemm.py:167-170); one thread per word.
template <int BITS>
__global__ __launch_bounds__(256) void group_dequantize_kernel(const uint32_t* __restrict__ packed,
                                                               const float* __restrict__ scales,
                                                               const float* __restrict__ biases, int64_t N,
                                                               int64_t K, int gs, float* __restrict__ w) {
    constexpr int PER = 32 / BITS;
    constexpr uint32_t L = (1u << BITS) - 1u;
    const int64_t words = N * K / PER;
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= words) return;
    const int64_t k0 = (id * PER) % K, n = (id * PER) / K;
    const int64_t gi = n * (K / gs) + k0 / gs;
    const float s = scales[gi];
    const float b = biases ? biases[gi] : 0.0f;
    const uint32_t word = packed[id];
    float out[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const float t = (float)((word >> (e * BITS)) & L) * s;
        out[e] = biases ? t + b : t;
    }
#pragma unroll
    for (int e = 0; e < PER; e += 4)
        *reinterpret_cast<vf4*>(w + id * PER + e) = vf4{out[e], out[e + 1], out[e + 2], out[e + 3]};
}

// ------------------------------------------- x . w_hat (quantized_matmul, transpose = false)
//
// y[m, k] = sum_n x[m, n] w_hat[n, k] for the packed w_hat[N, K] (groups along k): the product
// of quantized_matmul with transpose=false, and the input gradient of the transpose=true
// product, dX = dY dequant(W) (QuantizedMatmulBackward::apply, QuantizedMatmul.cpp:73-90).
// The group scale / bias change along the summed axis n, so there is no factoring of the
// sums as in the transpose=true kernel: each weight tile is dequantized into LDS exactly as
// group_dequantize_kernel writes it, fl32(fl32(c s) + b), and the kernel is a float32 tiled
// GEMM over it (128 x 128 outputs per 256-thread workgroup, 8 x 8 per thread, n in steps of
// 16, fused multiply-adds in n order).
constexpr int NT_T = 128, NT_K = 16, NT_R = NT_T / 16;

template <int BITS, bool XF32>
__global__ __launch_bounds__(256) void group_matmul_nt_kernel(const void* __restrict__ xv, int64_t ldx,
                                                              const uint32_t* __restrict__ packed,
                                                              const float* __restrict__ scales,
                                                              const float* __restrict__ biases,
                                                              const float* __restrict__ bias, void* __restrict__ yv,
                                                              int64_t ldy, int64_t M, int64_t N, int64_t K, int gs,
                                                              int relu, int hmode) {
    constexpr int PER = 32 / BITS;
    constexpr uint32_t L = (1u << BITS) - 1u;
    constexpr int WPR = NT_T / PER;  // packed words per tile row
    __shared__ __attribute__((aligned(16))) float xs[NT_K][NT_T + 4];  // row stride 16-byte aligned
    __shared__ __attribute__((aligned(16))) float ws[NT_K][NT_T];
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const int64_t G = K / gs, words_per_row = K / PER;
    const int64_t KT = (K + NT_T - 1) / NT_T, MT = (M + NT_T - 1) / NT_T;
    for (int64_t tile = blockIdx.x; tile < KT * MT; tile += gridDim.x) {
        const int64_t k0 = (tile % KT) * NT_T, m0 = (tile / KT) * NT_T;
        float acc[NT_R][NT_R] = {};
        // The next n-tile's activations and packed words (with their group scale / bias) are
        // loaded into registers while this tile's FMAs run, then dequantized into LDS.
        constexpr int XPT = NT_T * NT_K / 256, WPT = (NT_K * WPR + 255) / 256;
        float xq[XPT];
        uint32_t wq[WPT];
        float sq[WPT], bq[WPT];
        auto fetch = [&](int64_t n0) __attribute__((always_inline)) {
#pragma unroll
            for (int u = 0; u < XPT; ++u) {
                const int e = threadIdx.x + 256 * u;
                const int r = e / NT_K, kk = e % NT_K;
                const int64_t gm = m0 + r, gn = n0 + kk;
                float v = 0.0f;
                if (gm < M && gn < N) {
                    if constexpr (XF32) v = static_cast<const float*>(xv)[gm * ldx + gn];
                    else v = (float)static_cast<const _Float16*>(xv)[gm * ldx + gn];
                }
                xq[u] = v;
            }
#pragma unroll
            for (int u = 0; u < WPT; ++u) {
                const int e = threadIdx.x + 256 * u;
                const int r = e / WPR, wc = e % WPR;
                const int64_t gn = n0 + r, gk = k0 + (int64_t)wc * PER;
                wq[u] = 0u;
                sq[u] = 0.0f;
                bq[u] = 0.0f;
                if (e < NT_K * WPR && gn < N && gk < K) {  // K is a multiple of the group size: whole words
                    wq[u] = packed[gn * words_per_row + gk / PER];
                    const int64_t gi = gn * G + gk / gs;
                    sq[u] = round_to(scales[gi], hmode);
                    bq[u] = biases ? round_to(biases[gi], hmode) : 0.0f;
                }
            }
        };
        fetch(0);
        for (int64_t n0 = 0; n0 < N; n0 += NT_K) {
#pragma unroll
            for (int u = 0; u < XPT; ++u) {
                const int e = threadIdx.x + 256 * u;
                xs[e % NT_K][e / NT_K] = xq[u];
            }
#pragma unroll
            for (int u = 0; u < WPT; ++u) {
                const int e = threadIdx.x + 256 * u;
                if (e < NT_K * WPR) {
                    const int r = e / WPR, wc = e % WPR;
#pragma unroll
                    for (int q = 0; q < PER; ++q) {  // w_hat = fl32(fl32(c s) + b); 0 past N / K (s = 0)
                        const float t = (float)((wq[u] >> (q * BITS)) & L) * sq[u];
                        ws[r][wc * PER + q] = biases ? t + bq[u] : t;
                    }
                }
            }
            __syncthreads();
            if (n0 + NT_K < N) fetch(n0 + NT_K);
#pragma unroll
            for (int kk = 0; kk < NT_K; ++kk) {
                // this thread's NT_R consecutive rows and columns: 16-byte LDS reads
                float xr[NT_R], wr[NT_R];
#pragma unroll
                for (int i = 0; i < NT_R; i += 4) {
                    const vf4 v = *reinterpret_cast<const vf4*>(&xs[kk][ty * NT_R + i]);
                    xr[i] = v[0]; xr[i + 1] = v[1]; xr[i + 2] = v[2]; xr[i + 3] = v[3];
                }
#pragma unroll
                for (int j = 0; j < NT_R; j += 4) {
                    const vf4 v = *reinterpret_cast<const vf4*>(&ws[kk][tx * NT_R + j]);
                    wr[j] = v[0]; wr[j + 1] = v[1]; wr[j + 2] = v[2]; wr[j + 3] = v[3];
                }
#pragma unroll
                for (int i = 0; i < NT_R; ++i)
#pragma unroll
                    for (int j = 0; j < NT_R; ++j) acc[i][j] = fmaf(xr[i], wr[j], acc[i][j]);
            }
            __syncthreads();
        }
#pragma unroll
        for (int i = 0; i < NT_R; ++i) {
            const int64_t gm = m0 + ty * NT_R + i;
            if (gm >= M) continue;
#pragma unroll
            for (int j = 0; j < NT_R; ++j) {
                const int64_t gk = k0 + tx * NT_R + j;
                if (gk >= K) continue;
                const float v = wo_finish(acc[i][j], bias != nullptr, bias ? bias[gk] : 0.0f, relu, hmode);
                if constexpr (XF32) static_cast<float*>(yv)[gm * ldy + gk] = v;
                else static_cast<_Float16*>(yv)[gm * ldy + gk] = (_Float16)v;
            }
        }
    }
}

// ------------------------------------------------------------------ host side

struct WoPlan {
    int W, bpw;
    size_t lds;
};

// W waves split the T real k-blocks into equal runs of bpw blocks, bpw a multiple of the
// ring depth: the largest W (at most maxw) whose padded slots W * bpw stay within 1/8 of the
// fewest possible.
WoPlan wo_plan(int64_t K, int S, bool grouped, int maxw) {
    const int T = (int)((K + 32 * S - 1) / (32 * S));
    auto slots = [&](int W) {
        const int b = ((T + W - 1) / W + WO_RING - 1) / WO_RING * WO_RING;
        return (long)W * b;
    };
    long fewest = slots(1);
    for (int W = 2; W <= maxw; ++W) fewest = std::min(fewest, slots(W));
    int bestW = 1;
    for (int W = maxw; W >= 1; --W)
        if (slots(W) * 8 <= fewest * 9) {
            bestW = W;
            break;
        }
    const int bestB = (int)(slots(bestW) / bestW);
    WoPlan p{bestW, bestB, 0};
    const int TW = bestW * bestB;
    p.lds = sizeof(float) * ((size_t)bestW * 256 + (size_t)bestW * 64 + (grouped ? 2 * 16 * (size_t)TW : 0));
    return p;
}

// Workspace bytes of the pre-split activations: per 16-row tile and k-block, 64 lanes x 2 S
// vu4 plus 16 {2^-e, block sum} pairs.
size_t wo_prep_bytes(int64_t M, const WoPlan& p, int S) {
    const int64_t blocks = (M + 15) / 16 * (int64_t)p.W * p.bpw;
    return (size_t)blocks * (64 * 2 * S * sizeof(vu4) + 16 * sizeof(float2));
}

// Split-K layout of wo_gemv_sk_kernel: 64-column groups x K ranges of SK_RANGE_K.
struct SkPlan {
    int splits;
    int64_t groups;
};

SkPlan sk_plan(int64_t N, int64_t K) {
    return SkPlan{(int)((K + SK_RANGE_K - 1) / SK_RANGE_K), (N + 16 * SK_TILES - 1) / (16 * SK_TILES)};
}

// Workspace: the ranges' tile sums and activation row sums (none for a single range).
size_t sk_ws_bytes(const SkPlan& p) {
    if (p.splits <= 1) return 0;
    const size_t part = (size_t)p.splits * (size_t)p.groups * SK_TILES * 256 * sizeof(float);
    return ((part + 255) & ~(size_t)255) + (size_t)p.splits * 16 * sizeof(float);
}

// The split-K route: 3 <= M <= 16 with vector-aligned operands (the kernel's loads are
// unconditional 16-byte loads) and, when K is split, the workspace for the range sums.
constexpr int SK_MIN_M = 3, SK_MAX_M = 16;

// Row-major weights take the split-K kernel from 12 rows, or for weights over 16 MB (measured
// at K = N = 4096: M = 3..8 9.2-10 us on wo_gemv_kernel's in-workgroup split against 11.1-11.8
// here, equal from M = 12; at 11008 x 4096 this kernel is faster from M = 3: 20.5 against 24 us).
bool sk_preferred(const WoArgs& a) { return a.M >= 12 || (int64_t)a.N * a.K > ((int64_t)1 << 24); }

bool sk_fits(const WoArgs& a, bool xf32, int S, void* ws, size_t ws_bytes) {
    if (a.M < SK_MIN_M || a.M > SK_MAX_M) return false;
    const int eb = xf32 ? 4 : 2;
    if (!aligned16(a.w) || a.ldw_bytes % 16 || a.K % (8 * S) || a.K < 8 * S) return false;
    if (!aligned16(a.x) || (a.ldx * eb) % 16) return false;
    const SkPlan p = sk_plan(a.N, a.K);
    if (p.splits > 65535 || p.groups > ((int64_t)1 << 30)) return false;
    const size_t need = sk_ws_bytes(p);
    return need == 0 || (ws && aligned16(ws) && ws_bytes >= need);
}

template <int BITS, bool SIGNED, int S, bool GROUPED, bool PACKED = false>
int launch_sk(const WoArgs& a, bool xf32, hipStream_t st, void* ws) {
    const SkPlan p = sk_plan(a.N, a.K);
    WoSkArgs k{};
    k.w = a;
    k.splits = p.splits;
    if (p.splits > 1) {
        const size_t part = (size_t)p.splits * (size_t)p.groups * SK_TILES * 256 * sizeof(float);
        k.part = static_cast<float*>(ws);
        k.part_x = reinterpret_cast<float*>(static_cast<char*>(ws) + ((part + 255) & ~(size_t)255));
    }
    const dim3 grid((unsigned)p.groups, (unsigned)p.splits);
    if (xf32)
        hipLaunchKernelGGL((wo_gemv_sk_kernel<BITS, SIGNED, S, true, GROUPED, PACKED>), grid, dim3(64 * SK_WAVES), 0,
                           st, k);
    else
        hipLaunchKernelGGL((wo_gemv_sk_kernel<BITS, SIGNED, S, false, GROUPED, PACKED>), grid, dim3(64 * SK_WAVES), 0,
                           st, k);
    if (p.splits > 1) {
        const unsigned blocks = (unsigned)((p.groups * SK_TILES * 64 + 255) / 256);
        if (xf32)
            hipLaunchKernelGGL((wo_sk_reduce_kernel<true, GROUPED>), dim3(blocks), dim3(256), 0, st, k, (int)p.groups);
        else
            hipLaunchKernelGGL((wo_sk_reduce_kernel<false, GROUPED>), dim3(blocks), dim3(256), 0, st, k, (int)p.groups);
    }
    note_path(PACKED ? (p.splits > 1 ? "wo packed split-k" : "wo packed split-k single range")
                     : (p.splits > 1 ? "wo split-k" : "wo split-k single range"));
    return LQ_OK;
}

template <int BITS, bool SIGNED, int S, bool GROUPED, bool VEC>
int launch_wo(const WoPlan& p, WoArgs a, bool xf32, hipStream_t st, void* ws, size_t ws_bytes) {
    const dim3 grid((unsigned)((a.N + 15) / 16), (unsigned)((a.M + 15) / 16));
    const dim3 block(64 * p.W);
    const int TW = p.W * p.bpw;
    // The once-per-call split costs a launch of its own: it pays from 9 activation rows on
    // (M = 3..8 at 4096 x 4096: 9.3-10.5 us inline against 12.4 us with it; M = 16: 13.4
    // against 12.7 us).  Both routes give the same bits.
    if (xf32 && a.M > 8 && ws && ws_bytes >= wo_prep_bytes(a.M, p, S) && aligned16(ws)) {
        // split the activations once, then every workgroup reads the halves
        vu4* xp = static_cast<vu4*>(ws);
        float2* xm = reinterpret_cast<float2*>(xp + (int64_t)(a.M + 15) / 16 * TW * 64 * 2 * S);
        hipLaunchKernelGGL((wo_xprep_kernel<BITS, S>), dim3((unsigned)TW, (unsigned)((a.M + 15) / 16)), dim3(64), 0,
                           st, static_cast<const float*>(a.x), a.ldx, a.M, a.K, TW, xp, xm);
        a.xp = xp;
        a.xm = xm;
        hipLaunchKernelGGL((wo_gemv_kernel<BITS, SIGNED, S, true, GROUPED, VEC, true>), grid, block, p.lds, st, a);
        note_path("wo mfma presplit");
        return LQ_OK;
    } else if (xf32)
        hipLaunchKernelGGL((wo_gemv_kernel<BITS, SIGNED, S, true, GROUPED, VEC>), grid, block, p.lds, st, a);
    else
        hipLaunchKernelGGL((wo_gemv_kernel<BITS, SIGNED, S, false, GROUPED, VEC>), grid, block, p.lds, st, a);
    note_path("wo mfma");
    return LQ_OK;
}

// The VALU path: M <= 2, 16-byte aligned rows, at most 16 chunks per lane, staged rows fit
// 64 KB of LDS.  Returns false when the shape does not qualify.
template <int BITS, bool SIGNED, bool GROUPED>
bool launch_wv(WvArgs a, bool xf32, hipStream_t st) {
    constexpr int CK = 16 * 8 / BITS;
    if (a.M > 2) return false;
    const int64_t row_bytes = (int64_t)a.K * BITS / 8;
    if (row_bytes % 16) return false;
    a.NC = (int)(row_bytes / 16);
    const int Jn = (a.NC + 63) / 64;
    const int J = Jn <= 1 ? 1 : Jn <= 2 ? 2 : Jn <= 4 ? 4 : Jn <= 8 ? 8 : Jn <= 12 ? 12 : Jn <= 16 ? 16 : 0;
    if (J == 0) return false;
    a.Kpad = J * 64 * CK;
    {
        const int eb = xf32 ? 4 : 2;  // element bytes; a 4-element load needs 4 * eb alignment
        a.xvec = (reinterpret_cast<uintptr_t>(a.x) % (4 * eb) == 0) && ((a.ldx * eb) % (4 * eb) == 0);
    }
    const int MX = a.M;
    const int waves = a.N >= 4096 ? 16 : std::max(1, (a.N + 255) / 256);
    const size_t passes = ((size_t)MX * a.Kpad / 4 + 64 * waves - 1) / (64 * waves);
    const size_t lds = sizeof(float) * ((size_t)MX * a.Kpad +
                                        (GROUPED ? (size_t)MX * a.G : (size_t)MX + passes * waves * MX));
    if (lds > 64 * 1024) return false;
    const int64_t row_groups = (a.N + waves - 1) / waves;
    const bool persist = wv_persistent(GROUPED, MX, J);  // at most one workgroup per CU
    const dim3 grid((unsigned)(persist ? std::min<int64_t>(row_groups, device_cu_count()) : row_groups));
    const dim3 block(64 * waves);
    // (instantiated only for the chunk counts whose registers fit: group scales of 12+ chunks,
    // or of 8 chunks at 4 bits and two rows, would spill)
    auto go = [&](auto mx, auto xf, auto jv) {
        constexpr int MXV = decltype(mx)::value, JV = decltype(jv)::value;
        constexpr bool XV = decltype(xf)::value;
        constexpr bool fits = !GROUPED || (JV <= 8 && !(BITS == 4 && MXV == 2 && JV > 4));
        if constexpr (fits) {
            // group scales rounded to x's type: half x always, bfloat16 on request
            if constexpr (GROUPED && !XV)
                hipLaunchKernelGGL((wo_gemv_valu_kernel<BITS, SIGNED, GROUPED, MXV, XV, JV, LQ_ROUND_F16>), grid,
                                   block, lds, st, a);
            else if (GROUPED && a.hmode == LQ_ROUND_BF16)
                hipLaunchKernelGGL((wo_gemv_valu_kernel<BITS, SIGNED, GROUPED, MXV, XV, JV, LQ_ROUND_BF16>), grid,
                                   block, lds, st, a);
            else
                hipLaunchKernelGGL((wo_gemv_valu_kernel<BITS, SIGNED, GROUPED, MXV, XV, JV>), grid, block, lds, st, a);
            note_path("wo valu");
            return true;
        } else {
            return false;
        }
    };
    auto by_j = [&](auto mx, auto xf) {
        switch (J) {
            case 1: return go(mx, xf, std::integral_constant<int, 1>{});
            case 2: return go(mx, xf, std::integral_constant<int, 2>{});
            case 4: return go(mx, xf, std::integral_constant<int, 4>{});
            case 8: return go(mx, xf, std::integral_constant<int, 8>{});
            case 12: return go(mx, xf, std::integral_constant<int, 12>{});
            default: return go(mx, xf, std::integral_constant<int, 16>{});
        }
    };
    using T1 = std::integral_constant<int, 1>;
    using T2 = std::integral_constant<int, 2>;
    using F32 = std::integral_constant<bool, true>;
    using F16 = std::integral_constant<bool, false>;
    if (MX == 1) return xf32 ? by_j(T1{}, F32{}) : by_j(T1{}, F16{});
    return xf32 ? by_j(T2{}, F32{}) : by_j(T2{}, F16{});
}

constexpr int64_t WO_MAX_DIM = (int64_t)1 << 30;
constexpr size_t WO_MAX_LDS = 64 * 1024;

}  // namespace
}  // namespace lq

using namespace lq;

extern "C" {

size_t lq_gemv_w8_workspace_size(int64_t M, int64_t N, int64_t K) {
    if (M <= 2 || K <= 0 || M >= WO_MAX_DIM || K >= WO_MAX_DIM || N >= WO_MAX_DIM) return 0;  // VALU path
    const size_t prep = wo_prep_bytes(M, wo_plan(K, 2, false, wo_max_waves(2, true, false)), 2);
    if (M <= SK_MAX_M) return std::max(prep, sk_ws_bytes(sk_plan(std::max<int64_t>(N, 1), K)));
    return prep;
}

int lq_gemv_w8(const void* d_x, int x_dtype, int64_t ldx, const int8_t* d_W, int64_t ldw,
               const float* d_w_scale, const float* d_w_zero_point, const float* d_bias,
               void* d_y, int64_t ldy, int64_t M, int64_t N, int64_t K, int flags,
               void* d_workspace, size_t workspace_bytes, void* stream) {
    LQ_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M < WO_MAX_DIM && N < WO_MAX_DIM && K < WO_MAX_DIM,
               "lq_gemv_w8: bad shape");
    LQ_REQUIRE(x_dtype == LQ_F32 || x_dtype == LQ_F16, "lq_gemv_w8: x_dtype must be LQ_F32 or LQ_F16");
    LQ_REQUIRE((flags & ~LQ_EPI_RELU) == 0, "lq_gemv_w8: unknown flags");
    if (M == 0 || N == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_W && d_y && d_w_scale, "lq_gemv_w8: NULL pointer");
    LQ_REQUIRE(ldx >= K && ldw >= K && ldy >= N, "lq_gemv_w8: leading dimension too small");
    const bool xf32 = x_dtype == LQ_F32;
    const WoPlan p = wo_plan(std::max<int64_t>(K, 1), 2, false, wo_max_waves(2, xf32, false));
    WoArgs a{};
    a.x = d_x;
    a.ldx = ldx;
    a.w = reinterpret_cast<const uint8_t*>(d_W);
    a.ldw_bytes = ldw;
    a.w_scale = d_w_scale;
    a.w_zp = d_w_zero_point;
    a.bias = d_bias;
    a.y = d_y;
    a.ldy = ldy;
    a.relu = (flags & LQ_EPI_RELU) ? 1 : 0;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.bpw = p.bpw;
    hipStream_t st = as_stream(stream);
    if (M <= 2 && aligned16(d_W) && ldw % 16 == 0) {
        WvArgs v{};
        v.x = d_x; v.ldx = ldx; v.w = a.w; v.ldw_bytes = ldw; v.w_scale = d_w_scale;
        v.w_zp = d_w_zero_point; v.bias = d_bias; v.y = d_y; v.ldy = ldy; v.relu = a.relu;
        v.M = (int)M; v.N = (int)N; v.K = (int)K;
        if (launch_wv<8, true, false>(v, xf32, st)) return launch_status("lq_gemv_w8");
    }
    if (sk_preferred(a) && sk_fits(a, xf32, 2, d_workspace, workspace_bytes)) {
        const int rc = launch_sk<8, true, 2, false>(a, xf32, st, d_workspace);
        return rc ? rc : launch_status("lq_gemv_w8");
    }
    const bool vec = aligned16(d_W) && ldw % 16 == 0 && K % 16 == 0 && K >= 16 && aligned16(d_x) &&
                     ldx % (xf32 ? 4 : 8) == 0;
    if (vec) launch_wo<8, true, 2, false, true>(p, a, xf32, st, d_workspace, workspace_bytes);
    else launch_wo<8, true, 2, false, false>(p, a, xf32, st, d_workspace, workspace_bytes);
    return launch_status("lq_gemv_w8");
}

size_t lq_gemv_w8_packed_workspace_size(int64_t M, int64_t N, int64_t K) {
    if (M < 1 || M > SK_MAX_M || K <= 0 || K >= WO_MAX_DIM || N <= 0 || N >= WO_MAX_DIM) return 0;
    return sk_ws_bytes(sk_plan(N, K));
}

int lq_gemv_w8_packed(const void* d_x, int x_dtype, int64_t ldx, const int8_t* d_W_packed,
                      const float* d_w_scale, const float* d_w_zero_point, const float* d_bias, void* d_y,
                      int64_t ldy, int64_t M, int64_t N, int64_t K, int flags, void* d_workspace,
                      size_t workspace_bytes, void* stream) {
    LQ_REQUIRE(M >= 0 && N >= 0 && K >= 0 && N < WO_MAX_DIM && K < WO_MAX_DIM, "lq_gemv_w8_packed: bad shape");
    LQ_REQUIRE(M <= SK_MAX_M, "lq_gemv_w8_packed: at most 16 activation rows (use lq_gemv_w8)");
    LQ_REQUIRE(x_dtype == LQ_F32 || x_dtype == LQ_F16, "lq_gemv_w8_packed: x_dtype must be LQ_F32 or LQ_F16");
    LQ_REQUIRE((flags & ~LQ_EPI_RELU) == 0, "lq_gemv_w8_packed: unknown flags");
    if (M == 0 || N == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_W_packed && d_y && d_w_scale, "lq_gemv_w8_packed: NULL pointer");
    LQ_REQUIRE(ldx >= K && ldy >= N, "lq_gemv_w8_packed: leading dimension too small");
    const bool xf32 = x_dtype == LQ_F32;
    const int eb = xf32 ? 4 : 2;
    LQ_REQUIRE(K >= 16 && K % 16 == 0, "lq_gemv_w8_packed: K must be a positive multiple of 16");
    LQ_REQUIRE(aligned16(d_W_packed) && aligned16(d_x) && (ldx * eb) % 16 == 0,
               "lq_gemv_w8_packed: the weight, x and its rows must be 16-byte aligned");
    const size_t need = sk_ws_bytes(sk_plan(N, K));
    LQ_REQUIRE(need == 0 || (d_workspace && aligned16(d_workspace) && workspace_bytes >= need),
               "lq_gemv_w8_packed: workspace smaller than lq_gemv_w8_packed_workspace_size");
    WoArgs a{};
    a.x = d_x;
    a.ldx = ldx;
    a.w = reinterpret_cast<const uint8_t*>(d_W_packed);
    a.ldw_bytes = K;
    a.w_scale = d_w_scale;
    a.w_zp = d_w_zero_point;
    a.bias = d_bias;
    a.y = d_y;
    a.ldy = ldy;
    a.relu = (flags & LQ_EPI_RELU) ? 1 : 0;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    const int rc = launch_sk<8, true, 2, false, true>(a, xf32, as_stream(stream), d_workspace);
    return rc ? rc : launch_status("lq_gemv_w8_packed");
}

size_t lq_group_matmul_workspace_size(int64_t M, int64_t N, int64_t K, int group_size) {
    if (M <= 2 || K <= 0 || M >= WO_MAX_DIM || K >= WO_MAX_DIM || N >= WO_MAX_DIM) return 0;
    if (group_size != 32 && group_size != 64 && group_size != 128) return 0;
    const int S = group_size / 32;
    const size_t prep = wo_prep_bytes(M, wo_plan(K, S, true, wo_max_waves(S, true, true)), S);
    if (M <= SK_MAX_M) return std::max(prep, sk_ws_bytes(sk_plan(std::max<int64_t>(N, 1), K)));
    return prep;
}

int lq_group_matmul(const void* d_x, int x_dtype, int64_t ldx, const uint32_t* d_packed,
                    const float* d_scales, const float* d_biases, const float* d_bias, void* d_y,
                    int64_t ldy, int64_t M, int64_t N, int64_t K, int group_size, int bits,
                    int transpose, int flags, void* d_workspace, size_t workspace_bytes,
                    void* stream) {
    LQ_REQUIRE(M >= 0 && N >= 0 && K > 0 && M < WO_MAX_DIM && N < WO_MAX_DIM && K < WO_MAX_DIM,
               "lq_group_matmul: bad shape");
    LQ_REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
               "lq_group_matmul: group_size must be 32, 64 or 128");
    LQ_REQUIRE(bits == 4 || bits == 8, "lq_group_matmul: bits must be 4 or 8");
    LQ_REQUIRE(K % group_size == 0, "lq_group_matmul: K must be a multiple of group_size");
    LQ_REQUIRE(x_dtype == LQ_F32 || x_dtype == LQ_F16, "lq_group_matmul: x_dtype must be LQ_F32 or LQ_F16");
    LQ_REQUIRE((flags & ~(LQ_EPI_RELU | LQ_EPI_ROUND_BF16)) == 0, "lq_group_matmul: unknown flags");
    LQ_REQUIRE(!(flags & LQ_EPI_ROUND_BF16) || x_dtype == LQ_F32,
               "lq_group_matmul: LQ_EPI_ROUND_BF16 needs float32 x and y");
    // scales, group biases, layer bias and product in x's type (QuantizedMatmul.cpp:153-164)
    const int hmode = x_dtype == LQ_F16 ? LQ_ROUND_F16 : (flags & LQ_EPI_ROUND_BF16) ? LQ_ROUND_BF16 : LQ_ROUND_NONE;
    if (!transpose) {  // y[M, K] = x[M, N] w_hat[N, K]
        if (M == 0) return LQ_OK;
        LQ_REQUIRE(d_x && d_y && (N == 0 || (d_packed && d_scales)), "lq_group_matmul: NULL pointer");
        LQ_REQUIRE(ldx >= N && ldy >= K, "lq_group_matmul: leading dimension too small");
        const int64_t tiles = ((M + NT_T - 1) / NT_T) * ((K + NT_T - 1) / NT_T);
        const dim3 grid((unsigned)std::min<int64_t>(tiles, 1 << 20));
        const uint32_t* pk = N ? d_packed : nullptr;
        const float* gb = N ? d_biases : nullptr;
        const int relu = (flags & LQ_EPI_RELU) ? 1 : 0;
        hipStream_t st = as_stream(stream);
#define LQ_NT(B, XF)                                                                                           \
    hipLaunchKernelGGL((group_matmul_nt_kernel<B, XF>), grid, dim3(256), 0, st, d_x, ldx, pk, d_scales, gb, d_bias, \
                       d_y, ldy, M, N, K, group_size, relu, hmode)
        if (bits == 8) {
            if (x_dtype == LQ_F32) LQ_NT(8, true); else LQ_NT(8, false);
        } else {
            if (x_dtype == LQ_F32) LQ_NT(4, true); else LQ_NT(4, false);
        }
#undef LQ_NT
        return launch_status("lq_group_matmul");
    }
    if (M == 0 || N == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_packed && d_scales && d_y, "lq_group_matmul: NULL pointer");
    LQ_REQUIRE(ldx >= K && ldy >= N, "lq_group_matmul: leading dimension too small");
    LQ_REQUIRE(aligned16(d_packed), "lq_group_matmul: packed weights must be 16-byte aligned");
    const int S = group_size / 32;
    const bool xf32 = x_dtype == LQ_F32;
    const WoPlan p = wo_plan(K, S, true, wo_max_waves(S, xf32, true));
    if (p.lds > WO_MAX_LDS)
        return set_error(LQ_ERR_UNSUPPORTED, "lq_group_matmul: K too large for one workgroup's group scales");
    WoArgs a{};
    a.x = d_x;
    a.ldx = ldx;
    a.w = reinterpret_cast<const uint8_t*>(d_packed);
    a.ldw_bytes = K * bits / 8;
    a.w_scale = d_scales;
    a.g_bias = d_biases;
    a.bias = d_bias;
    a.y = d_y;
    a.ldy = ldy;
    a.relu = (flags & LQ_EPI_RELU) ? 1 : 0;
    a.hmode = hmode;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.G = (int)(K / group_size);
    a.bpw = p.bpw;
    hipStream_t st = as_stream(stream);
    if (M <= 2) {
        WvArgs v{};
        v.x = d_x; v.ldx = ldx; v.w = a.w; v.ldw_bytes = a.ldw_bytes; v.w_scale = d_scales;
        v.g_bias = d_biases; v.bias = d_bias; v.y = d_y; v.ldy = ldy; v.relu = a.relu; v.hmode = hmode;
        v.M = (int)M; v.N = (int)N; v.K = (int)K; v.G = a.G; v.gs = group_size;
        const bool ok = bits == 8 ? launch_wv<8, false, true>(v, xf32, st) : launch_wv<4, false, true>(v, xf32, st);
        if (ok) return launch_status("lq_group_matmul");
    }
    if (sk_preferred(a) && sk_fits(a, xf32, S, d_workspace, workspace_bytes)) {
        int rc;
        if (bits == 8) rc = S == 1 ? launch_sk<8, false, 1, true>(a, xf32, st, d_workspace)
                            : S == 2 ? launch_sk<8, false, 2, true>(a, xf32, st, d_workspace)
                                     : launch_sk<8, false, 4, true>(a, xf32, st, d_workspace);
        else rc = S == 1 ? launch_sk<4, false, 1, true>(a, xf32, st, d_workspace)
                  : S == 2 ? launch_sk<4, false, 2, true>(a, xf32, st, d_workspace)
                           : launch_sk<4, false, 4, true>(a, xf32, st, d_workspace);
        return rc ? rc : launch_status("lq_group_matmul");
    }
    const bool vec = aligned16(d_x) && ldx % (xf32 ? 4 : 8) == 0;
#define LQ_GM(B, SS)                                                          \
    do {                                                                      \
        if (vec) launch_wo<B, false, SS, true, true>(p, a, xf32, st, d_workspace, workspace_bytes);  \
        else launch_wo<B, false, SS, true, false>(p, a, xf32, st, d_workspace, workspace_bytes);     \
    } while (0)
    if (bits == 8) {
        if (S == 1) LQ_GM(8, 1); else if (S == 2) LQ_GM(8, 2); else LQ_GM(8, 4);
    } else {
        if (S == 1) LQ_GM(4, 1); else if (S == 2) LQ_GM(4, 2); else LQ_GM(4, 4);
    }
#undef LQ_GM
    return launch_status("lq_group_matmul");
}

int lq_group_quantize_f32(const float* d_w, int64_t N, int64_t K, int group_size, int bits,
                          uint32_t* d_packed, float* d_scales, float* d_biases, void* stream) {
    LQ_REQUIRE(N >= 0 && K >= 0, "lq_group_quantize_f32: bad shape");
    LQ_REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
               "lq_group_quantize_f32: group_size must be 32, 64 or 128");
    LQ_REQUIRE(bits == 4 || bits == 8, "lq_group_quantize_f32: bits must be 4 or 8");
    LQ_REQUIRE(K % group_size == 0, "lq_group_quantize_f32: K must be a multiple of group_size");
    if (N == 0 || K == 0) return LQ_OK;
    LQ_REQUIRE(d_w && d_packed && d_scales && d_biases, "lq_group_quantize_f32: NULL pointer");
    LQ_REQUIRE(aligned16(d_w), "lq_group_quantize_f32: weight must be 16-byte aligned");
    const int64_t groups = N * (K / group_size);
    const dim3 grid((unsigned)((groups + 255) / 256));
    if (bits == 8)
        hipLaunchKernelGGL(group_quantize_kernel<8>, grid, dim3(256), 0, as_stream(stream), d_w, N, K, group_size,
                           d_packed, d_scales, d_biases);
    else
        hipLaunchKernelGGL(group_quantize_kernel<4>, grid, dim3(256), 0, as_stream(stream), d_w, N, K, group_size,
                           d_packed, d_scales, d_biases);
    return launch_status("lq_group_quantize_f32");
}

int lq_group_dequantize_f32(const uint32_t* d_packed, const float* d_scales, const float* d_biases,
                            int64_t N, int64_t K, int group_size, int bits, float* d_w, void* stream) {
    LQ_REQUIRE(N >= 0 && K >= 0, "lq_group_dequantize_f32: bad shape");
    LQ_REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
               "lq_group_dequantize_f32: group_size must be 32, 64 or 128");
    LQ_REQUIRE(bits == 4 || bits == 8, "lq_group_dequantize_f32: bits must be 4 or 8");
    LQ_REQUIRE(K % group_size == 0, "lq_group_dequantize_f32: K must be a multiple of group_size");
    if (N == 0 || K == 0) return LQ_OK;
    LQ_REQUIRE(d_packed && d_scales && d_w, "lq_group_dequantize_f32: NULL pointer");
    LQ_REQUIRE(aligned16(d_w), "lq_group_dequantize_f32: output must be 16-byte aligned");
    const int64_t words = N * K * bits / 32;
    const dim3 grid((unsigned)((words + 255) / 256));
    if (bits == 8)
        hipLaunchKernelGGL(group_dequantize_kernel<8>, grid, dim3(256), 0, as_stream(stream), d_packed, d_scales,
                           d_biases, N, K, group_size, d_w);
    else
        hipLaunchKernelGGL(group_dequantize_kernel<4>, grid, dim3(256), 0, as_stream(stream), d_packed, d_scales,
                           d_biases, N, K, group_size, d_w);
    return launch_status("lq_group_dequantize_f32");
}

}  // extern "C"
