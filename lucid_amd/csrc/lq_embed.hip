// lq_embed.hip -- table lookups: Embedding and EmbeddingBag over an int8 or a float32 table.
//
// Lucid's quantized Embedding / EmbeddingBag (lucid/nn/quantized/sparse.py:140-143, 284-304)
// dequantize the whole per-row int8 table, then run the float lookup
// (lucid/_C/backend/cpu/methods/Sequence.cpp:520-552 embedding, :8-93 embedding_bag).  Here
// the lookup dequantizes only the rows it reads, in registers: a bag moves its indices' code
// rows and one float row out, never the float table.  The same kernels take a float32 table
// (scale NULL) for the float nn.Embedding / nn.EmbeddingBag.
//
// Per element: v = fl32(fl32(float(c) - z[row]) * s[row]) (lucid/quantization/_functional.py:293
// with ch_axis 0), or the float entry.  A bag walks its indices in order, as the CPU kernel:
//   sum   acc = 0; acc = acc + v           (with per_sample_weights: acc = acc + fl32(v * w),
//                                           the _bag_by_lookup composite, sparse.py:279-310)
//   mean  the sum, then acc / count when count > 0
//   max   acc = lowest float; if (v > acc) acc = v; an empty bag gives 0
// Indices equal to padding_idx are skipped and not counted (with per_sample_weights they add
// fl32(v * 0), as the composite's zero weight does).  An index outside [0, rows) reads no
// memory: its lookup row is NaN, and a bag that holds one is NaN -- the GPU policy of the
// reference (lucid/nn/functional/_index_checks.py: Metal isolates a bad index in the gather
// instead of reading it back); the Python layer refuses them first when strict.
//
// Work split: L lanes per output row (L a power of two <= 64 covering D in 4-element steps;
// 1-element steps when D % 4 != 0 or a pointer is misaligned); 256 / L rows per workgroup,
// grid-stride over rows.  HBM / L2 bound: the bytes are the looked-up code rows.
#include <hip/hip_runtime.h>

#include <float.h>

#include "lq_internal.h"

namespace lq {

constexpr int kEmbBlock = 256;
constexpr int KP = 4;  // bag indices gathered together (2: 198 us, 4: 182 us, 8: 198 us, 16: 294 us at 4M x 128, bags of 32)

struct EmbArgs {
    const void* table;
    int table_type;  // LQ_I8 or LQ_F32
    const float* scale;
    const float* zp;
    int64_t rows, D;
    const void* idx;
    int idx_type;  // LQ_I32 or LQ_I64
    int64_t n_idx;
    const void* offsets;  // NULL: fixed bags of bag_len
    int off_type;
    int64_t n_offsets, n_bags, bag_len;
    int mode;  // LQ_BAG_SUM / MEAN / MAX, or -1 for a plain lookup
    int64_t padding_idx;  // -1: none
    const float* psw;
    float* out;
    int lanes;  // L
};

__device__ __forceinline__ int64_t read_index(const void* p, int type, int64_t i) {
    return type == LQ_I64 ? static_cast<const int64_t*>(p)[i] : (int64_t) static_cast<const int32_t*>(p)[i];
}

// Elements [d, d + W) of table row r as floats (r in range, W = 4 or 1).
template <int W>
__device__ __forceinline__ void load_row(const EmbArgs& a, int64_t r, int64_t d, float (&v)[W]) {
    if (a.table_type == LQ_F32) {
        const float* p = static_cast<const float*>(a.table) + r * a.D + d;
        if constexpr (W == 4) {
            const vf4 q = *reinterpret_cast<const vf4*>(p);
            v[0] = q[0]; v[1] = q[1]; v[2] = q[2]; v[3] = q[3];
        } else {
            v[0] = p[0];
        }
    } else {
        const int8_t* p = static_cast<const int8_t*>(a.table) + r * a.D + d;
        float s, z;
        if (a.table_type == LQ_I8_QPAIR) {  // one 8-byte read of the row's {scale, zero point}
            const float2 q = reinterpret_cast<const float2*>(a.scale)[r];
            s = q.x;
            z = q.y;
        } else {
            s = a.scale[r];
            z = a.zp ? a.zp[r] : 0.0f;
        }
        int8_t c[W];
        if constexpr (W == 4) {
            const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
            __builtin_memcpy(c, &w, 4);
        } else {
            c[0] = p[0];
        }
#pragma unroll
        for (int e = 0; e < W; ++e) {
            const float dlt = (float)c[e] - z;
            v[e] = dlt * s;
        }
    }
}

template <int W>
__device__ __forceinline__ void store_out(float* p, const float (&v)[W]) {
    if constexpr (W == 4) *reinterpret_cast<vf4*>(p) = vf4{v[0], v[1], v[2], v[3]};
    else p[0] = v[0];
}

template <int W>
__global__ __launch_bounds__(kEmbBlock) void embed_kernel(EmbArgs a) {
    const int L = a.lanes;
    const int lane = threadIdx.x & (L - 1);
    const int64_t per_block = kEmbBlock / L;
    const int64_t out_rows = a.mode < 0 ? a.n_idx : a.n_bags;
    const float qnan = __builtin_nanf("");
    for (int64_t o = (int64_t)blockIdx.x * per_block + threadIdx.x / L; o < out_rows;
         o += (int64_t)gridDim.x * per_block) {
        float* orow = a.out + o * a.D;
        if (a.mode < 0) {  // plain lookup: padding_idx does not mask the forward
            const int64_t r = read_index(a.idx, a.idx_type, o);
            const bool ok = r >= 0 && r < a.rows;
            for (int64_t d = (int64_t)lane * W; d < a.D; d += (int64_t)L * W) {
                float v[W];
                if (ok) load_row<W>(a, r, d, v);
                else
#pragma unroll
                    for (int e = 0; e < W; ++e) v[e] = qnan;
                store_out<W>(orow + d, v);
            }
            continue;
        }
        int64_t k0, k1;
        if (a.offsets) {
            k0 = read_index(a.offsets, a.off_type, o);
            k1 = o + 1 < a.n_offsets ? read_index(a.offsets, a.off_type, o + 1) : a.n_idx;
        } else {
            k0 = o * a.bag_len;
            k1 = k0 + a.bag_len;
        }
        k0 = min(max(k0, (int64_t)0), a.n_idx);
        k1 = max(min(k1, a.n_idx), k0);
        for (int64_t d = (int64_t)lane * W; d < a.D; d += (int64_t)L * W) {
            float acc[W];
#pragma unroll
            for (int e = 0; e < W; ++e) acc[e] = a.mode == LQ_BAG_MAX ? -FLT_MAX : 0.0f;
            int count = 0;
            bool bad = false;
            // KP indices at a time: their row loads are all issued before the in-order folds,
            // so KP gathers are in flight per lane instead of one
            for (int64_t kb = k0; kb < k1; kb += KP) {
                int64_t r[KP];
#pragma unroll
                for (int j = 0; j < KP; ++j) r[j] = kb + j < k1 ? read_index(a.idx, a.idx_type, kb + j) : -1;
                float v[KP][W];
#pragma unroll
                for (int j = 0; j < KP; ++j) {
                    if (r[j] >= 0 && r[j] < a.rows) load_row<W>(a, r[j], d, v[j]);
                    else
#pragma unroll
                        for (int e = 0; e < W; ++e) v[j][e] = 0.0f;
                }
#pragma unroll
                for (int j = 0; j < KP; ++j) {
                    if (kb + j >= k1) break;
                    const bool pad = a.padding_idx >= 0 && r[j] == a.padding_idx;
                    if (pad && !a.psw) continue;
                    if (r[j] < 0 || r[j] >= a.rows) {
                        bad = true;
                        ++count;
                        continue;
                    }
                    if (a.psw) {
                        const float w = pad ? 0.0f : a.psw[kb + j];
#pragma unroll
                        for (int e = 0; e < W; ++e) {
                            const float t = v[j][e] * w;
                            acc[e] = acc[e] + t;
                        }
                    } else if (a.mode == LQ_BAG_MAX) {
#pragma unroll
                        for (int e = 0; e < W; ++e)
                            if (v[j][e] > acc[e]) acc[e] = v[j][e];
                    } else {
#pragma unroll
                        for (int e = 0; e < W; ++e) acc[e] = acc[e] + v[j][e];
                    }
                    if (!pad) ++count;
                }
            }
            if (a.mode == LQ_BAG_MAX && count == 0) {
#pragma unroll
                for (int e = 0; e < W; ++e) acc[e] = 0.0f;
            }
            if (a.mode == LQ_BAG_MEAN && count > 0) {
                const float cf = (float)count;
#pragma unroll
                for (int e = 0; e < W; ++e) acc[e] = acc[e] / cf;
            }
            if (bad) {
#pragma unroll
                for (int e = 0; e < W; ++e) acc[e] = qnan;
            }
            store_out<W>(orow + d, acc);
        }
    }
}

static int embed_launch(EmbArgs a, hipStream_t st) {
    const int es = a.table_type == LQ_F32 ? 4 : 1;
    const bool vec = a.D % 4 == 0 && ((uintptr_t)a.table & (uintptr_t)(4 * es - 1)) == 0 && aligned16(a.out);
    const int W = vec ? 4 : 1;
    const int64_t steps = (a.D + W - 1) / W;
    int L = 1;
    while (L < 64 && L < steps) L <<= 1;
    a.lanes = L;
    const int64_t out_rows = a.mode < 0 ? a.n_idx : a.n_bags;
    const int64_t per_block = kEmbBlock / L;
    int64_t blocks = (out_rows + per_block - 1) / per_block;
    if (blocks > 16384) blocks = 16384;
    if (vec) hipLaunchKernelGGL(embed_kernel<4>, dim3((unsigned)blocks), dim3(kEmbBlock), 0, st, a);
    else hipLaunchKernelGGL(embed_kernel<1>, dim3((unsigned)blocks), dim3(kEmbBlock), 0, st, a);
    return LQ_OK;
}

static int table_checks(const void* d_table, int table_type, const float* d_scale, int64_t rows, int64_t D,
                        int idx_type, const char* who) {
    (void)who;
    LQ_REQUIRE(rows >= 0 && D >= 0, "table lookup: negative table shape");
    LQ_REQUIRE(table_type == LQ_I8 || table_type == LQ_I8_QPAIR || table_type == LQ_F32,
               "table lookup: table_type must be LQ_I8, LQ_I8_QPAIR or LQ_F32");
    LQ_REQUIRE(table_type == LQ_F32 || d_scale, "table lookup: an int8 table needs its row scales");
    LQ_REQUIRE(table_type != LQ_I8_QPAIR || reinterpret_cast<uintptr_t>(d_scale) % 8 == 0,
               "table lookup: LQ_I8_QPAIR {scale, zero point} pairs must be 8-byte aligned");
    LQ_REQUIRE(idx_type == LQ_I32 || idx_type == LQ_I64, "table lookup: indices must be LQ_I32 or LQ_I64");
    LQ_REQUIRE(rows == 0 || D == 0 || d_table, "table lookup: NULL table");
    return LQ_OK;
}

}  // namespace lq

using namespace lq;

extern "C" {

int lq_embedding(const void* d_table, int table_type, const float* d_scale, const float* d_zero_point,
                 int64_t rows, int64_t D, const void* d_idx, int idx_type, int64_t n_idx, float* d_out,
                 void* stream) {
    int rc = table_checks(d_table, table_type, d_scale, rows, D, idx_type, "lq_embedding");
    if (rc != LQ_OK) return rc;
    LQ_REQUIRE(n_idx >= 0, "lq_embedding: n_idx < 0");
    if (n_idx == 0 || D == 0) return LQ_OK;
    LQ_REQUIRE(d_idx && d_out, "lq_embedding: NULL indices or output");
    EmbArgs a{d_table, table_type, d_scale, d_zero_point, rows, D, d_idx, idx_type, n_idx, nullptr, LQ_I64,
              0, 0, 0, -1, -1, nullptr, d_out, 1};
    embed_launch(a, as_stream(stream));
    return launch_status("lq_embedding");
}

int lq_embedding_bag(const void* d_table, int table_type, const float* d_scale, const float* d_zero_point,
                     int64_t rows, int64_t D, const void* d_idx, int idx_type, int64_t n_idx,
                     const void* d_offsets, int offsets_type, int64_t n_offsets, int include_last_offset,
                     int64_t bag_len, int mode, int64_t padding_idx, const float* d_per_sample_weights,
                     float* d_out, void* stream) {
    int rc = table_checks(d_table, table_type, d_scale, rows, D, idx_type, "lq_embedding_bag");
    if (rc != LQ_OK) return rc;
    LQ_REQUIRE(mode == LQ_BAG_SUM || mode == LQ_BAG_MEAN || mode == LQ_BAG_MAX, "lq_embedding_bag: bad mode");
    LQ_REQUIRE(!d_per_sample_weights || mode == LQ_BAG_SUM,
               "lq_embedding_bag: per_sample_weights is only supported for mode sum");
    LQ_REQUIRE(n_idx >= 0 && padding_idx >= -1, "lq_embedding_bag: n_idx < 0 or padding_idx < -1");
    int64_t n_bags;
    if (d_offsets) {
        LQ_REQUIRE(offsets_type == LQ_I32 || offsets_type == LQ_I64, "lq_embedding_bag: offsets must be LQ_I32 or LQ_I64");
        LQ_REQUIRE(n_offsets >= 0, "lq_embedding_bag: n_offsets < 0");
        n_bags = include_last_offset && n_offsets > 0 ? n_offsets - 1 : n_offsets;
    } else {
        LQ_REQUIRE(bag_len > 0 && n_idx % bag_len == 0, "lq_embedding_bag: without offsets n_idx must be a "
                                                        "multiple of bag_len > 0");
        n_bags = n_idx / bag_len;
    }
    if (n_bags == 0 || D == 0) return LQ_OK;
    LQ_REQUIRE(d_out && (n_idx == 0 || d_idx), "lq_embedding_bag: NULL indices or output");
    EmbArgs a{d_table, table_type, d_scale, d_zero_point, rows, D, d_idx, idx_type, n_idx, d_offsets,
              offsets_type, n_offsets, n_bags, bag_len, mode, padding_idx, d_per_sample_weights, d_out, 1};
    embed_launch(a, as_stream(stream));
    return launch_status("lq_embedding_bag");
}

}  // extern "C"
