// lq_gemm.hip -- W8A8 int8 GEMM on CDNA4 MFMA (v_mfma_i32_16x16x64_i8) with a fused
// zero-point / scale / bias / ReLU / requantize epilogue.
//
// Replaces the compute of Lucid's sidecar quantized Linear, which dequantizes the int8
// weight and runs an fp32 sgemm every call (lucid/nn/quantized/linear.py:206-215,
// lucid/nn/quantized/dynamic/linear.py:85-92 -> lucid/_C/nn/Linear.cpp:199 ->
// lucid/_C/backend/cpu/methods/Matmul.cpp:80-122).  Here the integer product is exact:
//
//   acc[m,n] = sum_k (A[m,k] - za) * (B[n,k] - zb[n])          (int32, wrap-free when it fits)
//            = sum_k A*B - za*bsum[n] - zb[n]*asum[m] + K*za*zb[n]
//   y        = fl32(fl32(float(acc) * fl32(sa[m] * sb[n])) + bias[n]), ReLU, then the output
//              kind (int32 / f32 / f16 / requantized codes / fake-quantized f32).
//
// Integer addition is associative, so the MFMA k-order, the tile split and split-K
// partial sums all give the same bits; the float epilogue is one IEEE op per step
// (compiled with -ffp-contract=off).
//
// Layout: A [M,K] and B [N,K] are both K-contiguous (Lucid's weight_int8 is [out, in]).
// The MFMA is fed B as its row operand and A as its column operand, so it produces C^T
// tiles: lane l holds four consecutive n of one m, which the epilogue stores as one vector.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <type_traits>

#include "lq_dma.h"
#include "lq_epilogue.h"
#include "lq_internal.h"

namespace lq {

typedef float v4f __attribute__((ext_vector_type(4)));

struct GemmArgs {
    const int8_t* A;
    const int8_t* B;
    void* C;
    int64_t lda, ldb, ldc;
    int M, N, K;
    const float* a_scale;
    const float* b_scale;
    int a_stride, b_stride;
    const float* a_zp;       // device scalar (integer valued) or null
    const float* b_zp;       // [N] (integer valued) or null
    const int32_t* b_sums;   // [N] sum_k B[n,k]; required when a_zp is set
    const int32_t* a_sums;   // [M] sum_k A[m,k]; required when b_zp is set
    const float* bias;       // [N] or null
    const float* out_scale;  // device scalar (requantizing kinds)
    const float* out_zp;     // device scalar or null
    int qmin, qmax;
    int out_kind;
    int relu;
    int gelu;                // float32 out: tanh GELU after the bias (LQ_EPI_GELU)
    int a_u8s8;              // A holds unsigned codes c as int8 (c - 128): the zero point shifts by 128
    int32_t* partial;        // split-K: [M,N] int32 accumulation buffer (zeroed)
    uint32_t* counters;      // split-K: one arrival counter per output tile (zeroed)
    int splits;              // split-K factor (1 = none)
    int2* extrema;           // float32 out, LDS-DMA kernels: per-workgroup extrema keys of the stored values
};

// ------------------------------------------------------------------ epilogue

__device__ __forceinline__ EpiParams epi_params(const GemmArgs& a) {
    EpiParams p;
    p.za = (a.a_zp ? (int)a.a_zp[0] : 0) - (a.a_u8s8 ? 128 : 0);
    p.has_za = a.a_zp != nullptr || a.a_u8s8;
    p.out_s = a.out_scale ? a.out_scale[0] : 1.0f;
    p.out_inv = 1.0f / p.out_s;
    p.out_z = a.out_zp ? a.out_zp[0] : 0.0f;
    p.g.lo = (float)a.qmin;
    p.g.hi = (float)a.qmax;
    p.g.lo_ties = (a.qmin == 0);
    p.g.hi_ties = false;
    return p;
}

// Zero-point corrected accumulator (two's-complement wrap; exact whenever it fits int32).
__device__ __forceinline__ int32_t corrected(int32_t raw, int m, int n, const GemmArgs& a,
                                             const EpiParams& p) {
    uint32_t acc = (uint32_t)raw;
    if (p.has_za) acc -= (uint32_t)p.za * (uint32_t)a.b_sums[n];
    if (a.b_zp) {
        const uint32_t zb = (uint32_t)(int)a.b_zp[n];
        acc -= zb * (uint32_t)a.a_sums[m];
        acc += (uint32_t)a.K * (uint32_t)p.za * zb;
    }
    return (int32_t)acc;
}

// Epilogue inputs of the four consecutive columns n..n+3 a lane owns, loaded once.
struct ColCtx {
    float sb[4], bias[4];
    int32_t bsum[4], zb[4];
    int n;
    bool vec;  // the four are in range and aligned for one vector store
};

// Epilogue inputs of one row m.
struct RowCtx {
    float sa;
    int32_t asum;
};

// Whether four consecutive outputs starting at column n can be one vector store.
__device__ __forceinline__ bool vec_store_ok(const GemmArgs& a, int n, int elem_bytes) {
    const bool base_ok = ((reinterpret_cast<uintptr_t>(a.C) & (uintptr_t)(4 * elem_bytes - 1)) == 0) &&
                         ((a.ldc & 3) == 0);
    return base_ok && (n + 3 < a.N);
}

template <int KIND>
__device__ __forceinline__ ColCtx load_cols(const GemmArgs& a, int n) {
    ColCtx c;
    c.n = n;
    c.vec = vec_store_ok(a, n, OutTraits<KIND>::bytes);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int nn = min(n + r, a.N - 1);  // clamped: out-of-range columns are never stored
        c.sb[r] = a.b_scale ? a.b_scale[(int64_t)nn * a.b_stride] : 1.0f;
        c.bias[r] = a.bias ? a.bias[nn] : 0.0f;
        c.bsum[r] = a.b_sums ? a.b_sums[nn] : 0;
        c.zb[r] = a.b_zp ? (int)a.b_zp[nn] : 0;
    }
    return c;
}

__device__ __forceinline__ RowCtx load_row(const GemmArgs& a, int m) {
    RowCtx r;
    const int mm = min(m, a.M - 1);  // clamped: rows past M are never stored
    r.sa = a.a_scale ? a.a_scale[(int64_t)mm * a.a_stride] : 1.0f;
    r.asum = a.b_zp ? a.a_sums[mm] : 0;
    return r;
}

// Four consecutive outputs C[m, c.n .. c.n+3] from raw accumulators.
template <int KIND>
__device__ __forceinline__ void epilogue4c(const GemmArgs& a, const EpiParams& p, const RowCtx& row,
                                           const ColCtx& c, int m, v4i raw) {
    if (m >= a.M) return;
    uint32_t out[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        uint32_t acc = (uint32_t)raw[r];  // zero-point correction, two's-complement wrap
        if (p.has_za) acc -= (uint32_t)p.za * (uint32_t)c.bsum[r];
        if (a.b_zp) {
            acc -= (uint32_t)c.zb[r] * (uint32_t)row.asum;
            acc += (uint32_t)a.K * (uint32_t)p.za * (uint32_t)c.zb[r];
        }
        out[r] = epi_one<KIND>((int32_t)acc, row.sa, c.sb[r], a.bias ? &c.bias[r] : nullptr, a.relu != 0, p,
                               a.gelu != 0);
    }
    const int64_t base = (int64_t)m * a.ldc + c.n;
    constexpr int b = OutTraits<KIND>::bytes;
    if (c.vec) {
        if (b == 4) {
            *reinterpret_cast<v4i*>(reinterpret_cast<uint32_t*>(a.C) + base) =
                v4i{(int)out[0], (int)out[1], (int)out[2], (int)out[3]};
        } else if (b == 2) {
            typedef int v2i __attribute__((ext_vector_type(2)));
            *reinterpret_cast<v2i*>(reinterpret_cast<uint16_t*>(a.C) + base) =
                v2i{(int)(out[0] | (out[1] << 16)), (int)(out[2] | (out[3] << 16))};
        } else {
            *reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(a.C) + base) =
                out[0] | (out[1] << 8) | (out[2] << 16) | (out[3] << 24);
        }
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (c.n + r < a.N) store_elem<KIND>(a.C, base + r, out[r]);
    }
}

template <int KIND>
__device__ __forceinline__ void epilogue4(const GemmArgs& a, const EpiParams& p, int m, int n, v4i raw) {
    if (m >= a.M) return;
    epilogue4c<KIND>(a, p, load_row(a, m), load_cols<KIND>(a, n), m, raw);
}


// ------------------------------------------------------------ tile scheduling

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2): block b
// runs on XCD b % 8.  Renumber so each XCD works on a contiguous run of tiles, then walk
// tiles in GROUP_M-tall bands so that run covers a compact block of A rows and B columns.
__device__ __forceinline__ void tile_of_block(int bid, int nblk, int tiles_m, int tiles_n, int& tm,
                                              int& tn) {
    constexpr int XCDS = 8, GROUP_M = 4;
    const int xcd = bid % XCDS, local = bid / XCDS;
    const int per = nblk / XCDS, rem = nblk % XCDS;
    const int t = xcd * per + (xcd < rem ? xcd : rem) + local;
    const int band = GROUP_M * tiles_n;
    const int first_m = (t / band) * GROUP_M;
    const int gsize = min(tiles_m - first_m, GROUP_M);
    const int in_band = t % band;
    tm = first_m + in_band % gsize;
    tn = in_band / gsize;
}

// ------------------------------------------------------- tiled MFMA main loop
//
// Block tile BM x BN, K staged 128 bytes at a time through double-buffered LDS.  Each LDS
// row holds the 128 K-bytes of one A (or B) row as eight 16-byte chunks, chunk c stored at
// slot c ^ (row & 7): the sixteen lanes that read one MFMA fragment (rows r..r+15, same
// chunk) then hit eight different 16-byte bank groups per half, and the eight lanes that
// write one row's chunks hit eight different slots.  One barrier per K stage: stage k+1
// is written into the other buffer while stage k is consumed.

constexpr int BK = 128;

template <int BM, int BN, int WAVES_M, int WAVES_N, int KIND>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_i8_tiled_kernel(GemmArgs a) {
    constexpr int T = 64 * WAVES_M * WAVES_N;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int FM = WM / 16, FN = WN / 16;
    constexpr int A_CH = BM * (BK / 16) / T;  // 16-byte chunks per thread per stage
    constexpr int B_CH = BN * (BK / 16) / T;
    static_assert(A_CH * T == BM * (BK / 16) && B_CH * T == BN * (BK / 16), "tile/threads mismatch");
    static_assert(FM >= 1 && FN >= 1, "wave tile smaller than one MFMA");

    __shared__ __attribute__((aligned(16))) int8_t As[2][BM * BK];
    __shared__ __attribute__((aligned(16))) int8_t Bs[2][BN * BK];

    const int tiles_m = (a.M + BM - 1) / BM, tiles_n = (a.N + BN - 1) / BN;
    const int ntiles = tiles_m * tiles_n;
    int tile_id = blockIdx.x, split = 0;
    if (a.splits > 1) {
        split = blockIdx.x / ntiles;
        tile_id = blockIdx.x % ntiles;
    }
    int tm, tn;
    tile_of_block(tile_id, ntiles, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    // K range of this split (whole BK stages).
    const int nk_total = (a.K + BK - 1) / BK;
    const int per_split = (nk_total + a.splits - 1) / a.splits;
    const int kt_begin = split * per_split;
    const int kt_end = min(nk_total, kt_begin + per_split);

    v4i ra[A_CH], rb[B_CH];
    auto gload = [&](int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int j = 0; j < A_CH; ++j) {
            const int q = tid + T * j, row = q >> 3, c = q & 7;
            const int gm = m0 + row, gk = k0 + c * 16;
            ra[j] = (gm < a.M && gk < a.K)
                        ? *reinterpret_cast<const v4i*>(a.A + (int64_t)gm * a.lda + gk)
                        : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < B_CH; ++j) {
            const int q = tid + T * j, row = q >> 3, c = q & 7;
            const int gn = n0 + row, gk = k0 + c * 16;
            rb[j] = (gn < a.N && gk < a.K)
                        ? *reinterpret_cast<const v4i*>(a.B + (int64_t)gn * a.ldb + gk)
                        : v4i{0, 0, 0, 0};
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int j = 0; j < A_CH; ++j) {
            const int q = tid + T * j, row = q >> 3, c = q & 7;
            *reinterpret_cast<v4i*>(&As[buf][row * BK + ((c ^ (row & 7)) << 4)]) = ra[j];
        }
#pragma unroll
        for (int j = 0; j < B_CH; ++j) {
            const int q = tid + T * j, row = q >> 3, c = q & 7;
            *reinterpret_cast<v4i*>(&Bs[buf][row * BK + ((c ^ (row & 7)) << 4)]) = rb[j];
        }
    };

    v4i acc[FN][FM];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    if (kt_begin < kt_end) {
        gload(kt_begin);
        lstore(0);
        __syncthreads();
        const int a_row0 = wm * WM + (lane & 15);
        const int b_row0 = wn * WN + (lane & 15);
        for (int kt = kt_begin; kt < kt_end; ++kt) {
            const int buf = (kt - kt_begin) & 1;
            const bool more = kt + 1 < kt_end;
            if (more) gload(kt + 1);
#pragma unroll
            for (int s = 0; s < BK / 64; ++s) {
                const int c = s * 4 + (lane >> 4);
                const int off = (c ^ (lane & 7)) << 4;
                v4i af[FM], bf[FN];
#pragma unroll
                for (int j = 0; j < FM; ++j)
                    af[j] = *reinterpret_cast<const v4i*>(&As[buf][(a_row0 + j * 16) * BK + off]);
#pragma unroll
                for (int i = 0; i < FN; ++i)
                    bf[i] = *reinterpret_cast<const v4i*>(&Bs[buf][(b_row0 + i * 16) * BK + off]);
#pragma unroll
                for (int i = 0; i < FN; ++i)
#pragma unroll
                    for (int j = 0; j < FM; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[i], af[j], acc[i][j], 0, 0, 0);
            }
            if (more) lstore(buf ^ 1);
            __syncthreads();
        }
    }

    if (a.splits > 1) {
        // Exact int32 partial sums: atomics commute, so the total is the same bits in any order.
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FM; ++j) {
                const int m = m0 + wm * WM + j * 16 + (lane & 15);
                const int n = n0 + wn * WN + i * 16 + (lane >> 4) * 4;
                if (m < a.M)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (n + r < a.N) atomicAdd(&a.partial[(int64_t)m * a.N + n + r], acc[i][j][r]);
            }
        // The last split to arrive at this tile runs the epilogue on the complete sums.
        __threadfence();
        __syncthreads();
        __shared__ int last;
        if (tid == 0) last = (atomicAdd(&a.counters[tile_id], 1u) == (unsigned)(a.splits - 1));
        __syncthreads();
        if (!last) return;
        __threadfence();
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FM; ++j) {
                const int m = m0 + wm * WM + j * 16 + (lane & 15);
                const int n = n0 + wn * WN + i * 16 + (lane >> 4) * 4;
                if (m < a.M)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[i][j][r] = (n + r < a.N)
                                           ? __hip_atomic_load(&a.partial[(int64_t)m * a.N + n + r],
                                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                           : 0;
            }
    }

    const EpiParams p = epi_params(a);
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) {
            const int m = m0 + wm * WM + j * 16 + (lane & 15);
            const int n = n0 + wn * WN + i * 16 + (lane >> 4) * 4;
            epilogue4<KIND>(a, p, m, n, acc[i][j]);
        }
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int NBUF_ = 2>
struct DmaTile {
    static constexpr int BK = 128, CPR = 8, KS = 2, NBUF = NBUF_;
    static constexpr int NW = WAVES_M * WAVES_N;
    static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    static constexpr int FM = WM / 16, FN = WN / 16;
    static constexpr int ROWS_PER_INSTR = 64 / CPR;
    static constexpr int A_I = BM / ROWS_PER_INSTR / NW;
    static constexpr int B_I = BN / ROWS_PER_INSTR / NW;
    static constexpr int LPS = A_I + B_I;  // copy instructions per wave per stage
    static constexpr int SB = (BM + BN) * BK;
    static constexpr int LDS_BYTES = NBUF * SB;
    static_assert(A_I * ROWS_PER_INSTR * NW == BM && B_I * ROWS_PER_INSTR * NW == BN, "copy split");
    static constexpr int NH = WN / 64;  // 64-column halves of the wave tile
    static_assert(WN % 64 == 0 && NH <= 2, "each lane owns 16 consecutive output columns of each 64-column half");
    static_assert(WM % 32 == 0, "fragment swizzle parity");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
};

// LDS stage buffers of the DMA main loop (a third buffer measured the same at 4096^3: the
// copies land within one stage; one round of 128x128 tiles takes three).
constexpr int GEMM_NBUF = 2;

// Scheduling pattern for one K step: R fragment reads (DS) spread over Q MFMAs, each read
// followed by its share of the MFMAs.
template <int R, int Q, int T = 0>
__device__ __forceinline__ void pin_reads_mfmas() {
    if constexpr (T < R) {
        constexpr int n = (T + 1) * Q / R - T * Q / R;
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
        if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x008, n, 0);  // n MFMAs
        pin_reads_mfmas<R, Q, T + 1>();
    }
}

// --------------------------------------------- LDS-DMA MFMA main loop (large M)
//
// The production path for M > 64 when K % 128 == 0.  Global -> LDS copies use the LDS-DMA
// form of buffer_load_dwordx4 (data goes straight to LDS, no staging registers): each wave
// instruction moves 1 KB = 8 rows x 128 K-bytes of A or B into the next stage's buffer.
// Buffer descriptors bound A and B to M*lda and N*ldb bytes, so rows past M or N read as
// zero (their outputs are never stored) and no per-row predicates are needed.
//
// A ring of NBUF LDS stages of BK = 128: stage kt+NBUF is issued right after the barrier
// that retires stage kt, and waited for (vmcnt) NBUF - 1 stages later.  Inside a stage the two 64-byte K steps
// ping-pong fragment registers: step s+1's fragments are read while step s's MFMAs run.
// The copy is issued from inline asm so the compiler neither tracks it nor inserts its own
// conservative vmcnt(0) in front of every LDS read (it cannot tell the stage buffers apart);
// the explicit vmcnt waits below are the synchronization.  Copies of stages past the end
// are clamped to the last stage (a valid address, landing in a buffer never read again),
// which keeps the steady-state loop free of branches; with a two-stage ring (wait =
// vmcnt(0)) the tail stages after the loop issue no copies at all.
//
// Output layout: B fragment i reads, in its lane row rho, the wave-tile row
// (rho / 4) * 16 + 4 i + rho % 4.  The MFMA's output lane l, register r then holds column
// 16 (l / 16) + 4 i + r, so over its four B fragments a lane owns 16 consecutive columns of
// each of its rows: the epilogue works from registers and stores 16-byte row segments
// (int8) directly, with no LDS round trip.  The per-column epilogue inputs are loaded
// after the main loop, so their registers do not compete with the fragment double buffer.

template <int BM, int BN, int WAVES_M, int WAVES_N, int NBUF, int KIND>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N)
__attribute__((amdgpu_waves_per_eu(WAVES_M * WAVES_N >= 8 ? 2 : 1))) void gemm_i8_dma_kernel(GemmArgs a) {
    typedef DmaTile<BM, BN, WAVES_M, WAVES_N, NBUF> P;
    static_assert(NBUF >= 2 && (NBUF - 1) * P::LPS < 64, "stage ring");
    constexpr int BK = P::BK, NW = P::NW, WM = P::WM, WN = P::WN, FM = P::FM, FN = P::FN, NH = P::NH;
    constexpr int RPI = P::ROWS_PER_INSTR, A_I = P::A_I, B_I = P::B_I, SB = P::SB;
    constexpr bool INT_CODES = KIND == LQ_OUT_Q8 || KIND == LQ_OUT_QU8 || KIND == LQ_OUT_Q16 || KIND == LQ_OUT_QU8S8;
    // Stage ring, then the epilogue inputs (EPI_ARR bytes each: column scales, bias, column code
    // sums, row scales).
    constexpr int EPI_ARR = 1024;
    static_assert(BM <= EPI_ARR / 4 && BN <= EPI_ARR / 4 && P::LDS_BYTES + 4 * EPI_ARR <= 160 * 1024, "epilogue LDS");
    __shared__ __attribute__((aligned(1024))) int8_t lds[P::LDS_BYTES + 4 * EPI_ARR];

    const int tiles_m = (a.M + BM - 1) / BM, tiles_n = (a.N + BN - 1) / BN;
    int tm, tn;
    tile_of_block(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int nk = a.K / BK;
    const EpiParams p = epi_params(a);

    // Epilogue inputs of a whole tile (both dimensions in range, unit-stride scales, 16-byte
    // aligned arrays) are copied into LDS before the main loop, one LDS-DMA per array (waves 0-3),
    // so the epilogue reads them from LDS instead of waiting for global loads after the loop.
    // These copies are older than every stage copy, so the prologue's vmcnt wait covers them
    // and its barrier publishes them.
    auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    const bool pre = nk > 0 && n0 + BN <= a.N && m0 + BM <= a.M && a.b_scale && a.b_stride == 1 &&
                     al16(a.b_scale) && a.a_scale && a.a_stride == 1 && al16(a.a_scale) &&
                     (!a.bias || al16(a.bias)) && (!p.has_za || al16(a.b_sums));
    const uint32_t lds_epi = (uint32_t)reinterpret_cast<uintptr_t>(lds) + P::LDS_BYTES;
    if (pre && wave < 4) {
        const void* src = wave == 0 ? (const void*)a.b_scale
                          : wave == 1 ? (const void*)a.bias
                          : wave == 2 ? (p.has_za ? (const void*)a.b_sums : nullptr)
                                      : (const void*)a.a_scale;
        const int first = wave == 3 ? m0 : n0, count = wave == 3 ? a.M : a.N;
        if (src) {
            const v4i r = buffer_rsrc(src, (uint32_t)count * 4u);
            lds_dma16(r, (uint32_t)lane * 16u, (uint32_t)first * 4u, lds_epi + wave * EPI_ARR);
        }
    }

    const v4i ra = buffer_rsrc(a.A, (uint32_t)((int64_t)a.M * a.lda));
    const v4i rb = buffer_rsrc(a.B, (uint32_t)((int64_t)a.N * a.ldb));
    // Lane l of a copy moves chunk slot l % 8 of row l / 8 of its 8-row block: the global
    // chunk (l % 8) ^ dma_swz(row).
    uint32_t a_off[A_I], b_off[B_I];
    {
        const int rl = lane >> 3, slot = lane & 7;
#pragma unroll
        for (int j = 0; j < A_I; ++j) {
            const int r = (j * NW + wave) * RPI + rl;
            a_off[j] = (uint32_t)(m0 + r) * (uint32_t)a.lda + (uint32_t)((slot ^ dma_swz(r)) * 16);
        }
#pragma unroll
        for (int j = 0; j < B_I; ++j) {
            const int r = (j * NW + wave) * RPI + rl;
            b_off[j] = (uint32_t)(n0 + r) * (uint32_t)a.ldb + (uint32_t)((slot ^ dma_swz(r)) * 16);
        }
    }
    const uint32_t lds_base = (uint32_t)reinterpret_cast<uintptr_t>(lds);
    auto issue = [&](int buf, int kt) __attribute__((always_inline)) {
        const uint32_t k0 = (uint32_t)(min(kt, nk - 1) * BK);
        const uint32_t sb = lds_base + buf * SB;
#pragma unroll
        for (int j = 0; j < A_I; ++j) lds_dma16(ra, a_off[j], k0, sb + (j * NW + wave) * RPI * BK);
#pragma unroll
        for (int j = 0; j < B_I; ++j) lds_dma16(rb, b_off[j], k0, sb + BM * BK + (j * NW + wave) * RPI * BK);
    };
    // Fragment addresses.  A fragment j: rows wm*WM + 16 j + rho, rho = lane % 16; B fragment i:
    // rows wn*WN + 64 (i / 4) + (rho / 4) * 16 + 4 (i % 4) + rho % 4.  Logical chunk of K step s:
    // 4 s + lane / 16.
    // The swizzle of an A row depends on rho and the parity of j, that of a B row on rho and
    // the parity of i; the K step flips chunk bit 2.  So two base offsets per operand, with
    // bit 6 (chunk bit 2) toggled by s ^ parity.
    const int rho = lane & 15, c0 = lane >> 4;
    const int a_base = (wm * WM + rho) * BK + ((c0 ^ (rho & 7)) << 4);
    const int b_row = wn * WN + (rho >> 2) * 16 + (rho & 3);
    const int b_base = BM * BK + b_row * BK + ((c0 ^ dma_swz(b_row)) << 4);
    v4i F0[FM + FN], F1[FM + FN];
    auto read_frags = [&](v4i* f, int buf, int s) __attribute__((always_inline)) {
        const int8_t* sbuf = lds + buf * SB;
#pragma unroll
        for (int j = 0; j < FM; ++j)
            f[j] = *reinterpret_cast<const v4i*>(sbuf + (a_base ^ (((s ^ j) & 1) << 6)) + j * 16 * BK);
#pragma unroll
        for (int i = 0; i < FN; ++i)
            f[FM + i] = *reinterpret_cast<const v4i*>(sbuf + (b_base ^ (((s ^ i) & 1) << 6)) + (i & 3) * 4 * BK +
                                                      (i >> 2) * 64 * BK);
    };
    v4i acc[FN][FM];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = v4i{0, 0, 0, 0};
    auto mfmas = [&](const v4i* f) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FM; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(f[FM + i], f[j], acc[i][j], 0, 0, 0);
    };
    // The scheduler would otherwise place each fragment read right before its first MFMA
    // (and wait for it there); pin the order instead: the next step's FM + FN reads spread
    // over this step's FM * FN MFMAs, one read ahead of each run of MFMAs.
    auto pin_order = [&]() __attribute__((always_inline)) { pin_reads_mfmas<FM + FN, FM * FN>(); };
    // One stage in buffer B (compile time), ending with the switch to the other buffer.
    auto stage = [&](auto bc, int kt, bool last, auto tail_c) __attribute__((always_inline)) {
        constexpr int B = decltype(bc)::value;
        constexpr bool TAIL = decltype(tail_c)::value;
        read_frags(F1, B, 1);
        mfmas(F0);
        pin_order();
        if (!last) {
            wait_vmcnt<(NBUF - 2) * P::LPS>();  // stage kt+1 has landed (kt+2.. may be in flight)
            block_barrier();  // ... in every wave, and every wave is done reading stage kt
            if constexpr (!TAIL || NBUF > 2) issue(B, kt + NBUF);
            read_frags(F0, (B + 1) % NBUF, 0);
        }
        mfmas(F1);
        if (!last) pin_order();
    };

    if (nk > 0) {
#pragma unroll
        for (int j = 0; j < NBUF; ++j) issue(j, j);
        wait_vmcnt<(NBUF - 1) * P::LPS>();
        block_barrier();
        read_frags(F0, 0, 0);
        int kt = 0;
        for (; kt + NBUF < nk; kt += NBUF) {
            [&]<int... Bs>(std::integer_sequence<int, Bs...>) {
                (stage(std::integral_constant<int, Bs>(), kt + Bs, false, std::false_type()), ...);
            }(std::make_integer_sequence<int, NBUF>());
        }
        [&]<int... Bs>(std::integer_sequence<int, Bs...>) {
            ((kt + Bs < nk ? stage(std::integral_constant<int, Bs>(), kt + Bs, kt + Bs + 1 == nk, std::true_type())
                           : void()),
             ...);
        }(std::make_integer_sequence<int, NBUF>());
    }
    // Epilogue inputs: from LDS when the prologue copied them there, else loaded after the main
    // loop so their registers (52 per lane) do not compete with the fragment double buffer:
    // this lane's 16 columns and FM rows, as 16-byte loads when the 16 columns are in range and
    // the arrays aligned.
    const int mr0 = m0 + wm * WM + (lane & 15);
    // Both halves' column inputs and the row scales are loaded (and waited for) before any
    // output store: stores count in vmcnt too, so a wait placed after the first half's stores
    // would also wait for those stores to drain.
    float csbs[NH][16], cbiass[NH][16];
    int32_t czabs[NH][16];  // za * bsum[n]
    static_for<NH>([&](auto h_c) __attribute__((always_inline)) {
        constexpr int HF = decltype(h_c)::value;
        const int nc0 = n0 + wn * WN + HF * 64 + (lane >> 4) * 16;
        float* csb = csbs[HF];
        float* cbias = cbiass[HF];
        int32_t* czab = czabs[HF];
        if (pre) {
            const float* le = reinterpret_cast<const float*>(lds + P::LDS_BYTES);
            const int c = nc0 - n0;
    #pragma unroll
            for (int h = 0; h < 4; ++h) {
                const v4f v = *reinterpret_cast<const v4f*>(le + c + 4 * h);
                const v4f w = a.bias ? *reinterpret_cast<const v4f*>(le + EPI_ARR / 4 + c + 4 * h) : v4f{0, 0, 0, 0};
                const v4i u = p.has_za ? *reinterpret_cast<const v4i*>(le + EPI_ARR / 2 + c + 4 * h) : v4i{0, 0, 0, 0};
    #pragma unroll
                for (int e = 0; e < 4; ++e) {
                    csb[4 * h + e] = v[e];
                    cbias[4 * h + e] = w[e];
                    czab[4 * h + e] = (int32_t)((uint32_t)p.za * (uint32_t)u[e]);
                }
            }
        } else {
            const bool cols_vec = nc0 + 16 <= a.N;
            auto vec_ok = [&](const void* ptr) { return cols_vec && (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
            if (a.b_scale && a.b_stride == 1 && vec_ok(a.b_scale)) {
    #pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const v4f v = *reinterpret_cast<const v4f*>(a.b_scale + nc0 + 4 * h);
                    csb[4 * h] = v[0], csb[4 * h + 1] = v[1], csb[4 * h + 2] = v[2], csb[4 * h + 3] = v[3];
                }
            } else {
    #pragma unroll
                for (int q = 0; q < 16; ++q)
                    csb[q] = a.b_scale ? a.b_scale[(int64_t)min(nc0 + q, a.N - 1) * a.b_stride] : 1.0f;
            }
            if (a.bias && vec_ok(a.bias)) {
    #pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const v4f v = *reinterpret_cast<const v4f*>(a.bias + nc0 + 4 * h);
                    cbias[4 * h] = v[0], cbias[4 * h + 1] = v[1], cbias[4 * h + 2] = v[2], cbias[4 * h + 3] = v[3];
                }
            } else {
    #pragma unroll
                for (int q = 0; q < 16; ++q) cbias[q] = a.bias ? a.bias[min(nc0 + q, a.N - 1)] : 0.0f;
            }
            if (p.has_za && vec_ok(a.b_sums)) {
    #pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const v4i v = *reinterpret_cast<const v4i*>(a.b_sums + nc0 + 4 * h);
    #pragma unroll
                    for (int e = 0; e < 4; ++e) czab[4 * h + e] = (int32_t)((uint32_t)p.za * (uint32_t)v[e]);
                }
            } else {
    #pragma unroll
                for (int q = 0; q < 16; ++q)
                    czab[q] = p.has_za ? (int32_t)((uint32_t)p.za * (uint32_t)a.b_sums[min(nc0 + q, a.N - 1)]) : 0;
            }
        }
    });
    float rsa[FM];
    static_for<FM>([&](auto j_c) __attribute__((always_inline)) {
        constexpr int j = decltype(j_c)::value;
        if (pre) {
            rsa[j] = reinterpret_cast<const float*>(lds + P::LDS_BYTES + 3 * EPI_ARR)[mr0 - m0 + j * 16];
        } else {
            const int mm = min(mr0 + j * 16, a.M - 1);
            rsa[j] = a.a_scale ? a.a_scale[(int64_t)mm * a.a_stride] : 1.0f;
        }
    });

    wait_vmcnt<0>();  // no copy may still target LDS when the workgroup ends

    // One 64-column half HF of the wave tile at a time: acc[4 HF + i][j][r] is
    // C[mr0 + 16 j][nc0 + 4 i + r].
    int32_t ext_min = KEY_POS_INF, ext_max = KEY_NEG_INF;  // float32 out with a.extrema
    auto epilogue_half = [&](auto h_c) __attribute__((always_inline)) {
        constexpr int HF = decltype(h_c)::value;
        const int ncw = n0 + wn * WN + HF * 64;  // first column of this 64-column half
        const int nc0 = ncw + (lane >> 4) * 16;
        const float* csb = csbs[HF];
        const float* cbias = cbiass[HF];
        const int32_t* czab = czabs[HF];

        // Epilogue from registers.  Every lane computes (rows past M hold zeros), so the
        // cross-lane exchange below sees whole rows; only the stores are guarded.
        constexpr int OB = OutTraits<KIND>::bytes;
        const bool vec = (reinterpret_cast<uintptr_t>(a.C) % 16 == 0) && ((a.ldc * OB) % 16 == 0) &&
                         (ncw + 64 <= a.N);
        CodeClamp cc{};
        if (INT_CODES) cc = code_clamp<KIND>(a.qmin, a.qmax);
        const bool has_bias = a.bias != nullptr, relu = a.relu != 0;

        // Stores of one row's 16 outputs (bits of the output type in out[]).
        auto store_row = [&](int j, const uint32_t* out) __attribute__((always_inline)) {
            const int m = mr0 + j * 16;
            const bool row_ok = m < a.M;
            if (vec) {
                if (OB == 1) {
                    v4i w;
    #pragma unroll
                    for (int d = 0; d < 4; ++d) w[d] = (int)pack_low_bytes(out + 4 * d);
                    if (row_ok) *reinterpret_cast<v4i*>(reinterpret_cast<uint8_t*>(a.C) + (int64_t)m * a.ldc + nc0) = w;
                } else if (OB == 2) {
    #pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        v4i w;
    #pragma unroll
                        for (int d = 0; d < 4; ++d)
                            w[d] = (int)((out[8 * h + 2 * d] & 0xffffu) | (out[8 * h + 2 * d + 1] << 16));
                        if (row_ok)
                            *reinterpret_cast<v4i*>(reinterpret_cast<uint16_t*>(a.C) + (int64_t)m * a.ldc + nc0 + 8 * h) = w;
                    }
                } else {
                    // 4-byte outputs: lane group g = lane / 16 holds 16-byte pieces h = 0..3 of
                    // columns 16 g + 4 h.  A 4x4 transpose across (g, h) -- permlane32 swaps of
                    // pieces (0,2), (1,3), then permlane16 swaps of (0,1), (2,3), all among lanes
                    // of the same row -- leaves piece (h, g) in lane group g, register h, so
                    // store h covers 64 contiguous bytes of the row.
                    uint32_t v[4][4];
    #pragma unroll
                    for (int h = 0; h < 4; ++h)
    #pragma unroll
                        for (int d = 0; d < 4; ++d) v[h][d] = out[4 * h + d];
    #pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        auto s02 = __builtin_amdgcn_permlane32_swap(v[0][d], v[2][d], false, false);
                        auto s13 = __builtin_amdgcn_permlane32_swap(v[1][d], v[3][d], false, false);
                        v[0][d] = s02[0], v[2][d] = s02[1], v[1][d] = s13[0], v[3][d] = s13[1];
                        auto s01 = __builtin_amdgcn_permlane16_swap(v[0][d], v[1][d], false, false);
                        auto s23 = __builtin_amdgcn_permlane16_swap(v[2][d], v[3][d], false, false);
                        v[0][d] = s01[0], v[1][d] = s01[1], v[2][d] = s23[0], v[3][d] = s23[1];
                    }
                    const int64_t rb0 = (int64_t)m * a.ldc + ncw + (lane >> 4) * 4;
    #pragma unroll
                    for (int h = 0; h < 4; ++h)
                        if (row_ok)
                            *reinterpret_cast<v4i*>(reinterpret_cast<uint32_t*>(a.C) + rb0 + 16 * h) =
                                v4i{(int)v[h][0], (int)v[h][1], (int)v[h][2], (int)v[h][3]};
                }
            } else if (row_ok) {
                const int64_t base = (int64_t)m * a.ldc + nc0;
    #pragma unroll
                for (int q = 0; q < 16; ++q)
                    if (nc0 + q < a.N) store_elem<KIND>(a.C, base + q, out[q]);
            }
        };

        // Integer codes, fast form.  When the output scale's reciprocal is finite and positive,
        // the zero point integral and small, every scale and bias of this wave finite and
        // max|sa| * max|sb| small enough that float(acc) * s cannot overflow, y is always finite
        // (y * inv may be infinite, never NaN), and the code clamp(rne(y * inv) + z, lo, hi)
        // equals zi + med3(rne(y * inv), lo - zi, hi - zi).  The rounding is rne_bits (one add
        // whose float bits are RNE_MAGIC_BITS + rne(t), ordered outside the exact range), so the
        // clamp runs on the bits against bounds shifted by RNE_MAGIC_BITS and the low byte or
        // halfword of the result is the code: |zi| < 2^21 keeps the shifted bounds inside the
        // exact window.  ReLU (y <= 0 -> 0, so the code of z) folds into the lower bound:
        // rne(y * inv) <= 0 exactly when y <= 0.  The stored byte of QU8S8 is c - 128.
        bool fast_int = false;
        if constexpr (INT_CODES) {
            const float zf = p.out_z;
            bool ok = a.b_zp == nullptr && p.out_inv > 0.0f && p.out_inv < 3.0e38f && zf == __builtin_rintf(zf) &&
                      __builtin_fabsf(zf) < 2097152.0f;
            float amax = 0.0f, bmax = 0.0f;
    #pragma unroll
            for (int j = 0; j < FM; ++j) amax = __builtin_fmaxf(amax, __builtin_fabsf(rsa[j]));
    #pragma unroll
            for (int q = 0; q < 16; ++q) {
                bmax = __builtin_fmaxf(bmax, __builtin_fabsf(csb[q]));
                ok = ok && __builtin_isfinite(cbias[q]);
            }
            // fmaxf ignores NaN: test the maxima and every scale for finiteness
    #pragma unroll
            for (int j = 0; j < FM; ++j) ok = ok && __builtin_isfinite(rsa[j]);
    #pragma unroll
            for (int q = 0; q < 16; ++q) ok = ok && __builtin_isfinite(csb[q]);
            ok = ok && amax < 1.0e14f && bmax < 1.0e14f && amax * bmax < 1.0e28f;
            fast_int = __all(ok);
        }
        if constexpr (INT_CODES) {
            if (fast_int) {
                const int zi = (int)p.out_z;
                int L = cc.lo - zi, H = cc.hi - zi;
                if (relu) L = max(L, 0);
                L = min(L, H);  // med3(x, L, H) = min(max(x, L), H) needs L <= H
                const int Lm = L + RNE_MAGIC_BITS, Hm = H + RNE_MAGIC_BITS;
                const int shift = zi - (KIND == LQ_OUT_QU8S8 ? 128 : 0);
                // ZA / SHIFT off when the activation zero point / the code shift are zero:
                // two VALU ops fewer per element.
                auto rows = [&](auto bias_c, auto za_c, auto shift_c) __attribute__((always_inline)) {
                    constexpr bool BIAS = decltype(bias_c)::value, ZA = decltype(za_c)::value;
                    constexpr bool SHIFT = decltype(shift_c)::value;
                    static_for<FM>([&](auto j_c) __attribute__((always_inline)) {
                        constexpr int j = decltype(j_c)::value;
                        uint32_t out[16];
    #pragma unroll
                        for (int q = 0; q < 16; ++q) {
                            int32_t accq = acc[4 * HF + (q >> 2)][j][q & 3];
                            if (ZA) accq = (int32_t)((uint32_t)accq - (uint32_t)czab[q]);
                            const float sc = rsa[j] * csb[q];
                            float y = (float)accq * sc;
                            if (BIAS) y = y + cbias[q];
                            int32_t c = med3_i32(rne_bits(y * p.out_inv), Lm, Hm);
                            if (SHIFT) c += shift;
                            out[q] = (uint32_t)c;  // low byte / halfword: the code
                        }
                        store_row(j, out);
                    });
                };
                auto rows_za = [&](auto bias_c) __attribute__((always_inline)) {
                    if (p.has_za) {
                        if (shift != 0) rows(bias_c, std::true_type{}, std::true_type{});
                        else rows(bias_c, std::true_type{}, std::false_type{});
                    } else {
                        if (shift != 0) rows(bias_c, std::false_type{}, std::true_type{});
                        else rows(bias_c, std::false_type{}, std::false_type{});
                    }
                };
                if (has_bias) rows_za(std::true_type{});
                else rows_za(std::false_type{});
                return;
            }
        }
        // General form (any zero points, non-finite inputs, non-integral output zero point, and
        // the float kinds): bias and ReLU resolved outside the element loop.
        auto rows_general = [&](auto bias_c, auto relu_c) __attribute__((always_inline)) {
            constexpr bool BIAS = decltype(bias_c)::value, RELU = decltype(relu_c)::value;
            static_for<FM>([&](auto j_c) __attribute__((always_inline)) {
                constexpr int j = decltype(j_c)::value;
                const int m = mr0 + j * 16;
                int32_t asum = 0;
                if (a.b_zp) asum = a.a_sums[min(m, a.M - 1)];
                uint32_t out[16];
    #pragma unroll
                for (int q = 0; q < 16; ++q) {
                    uint32_t accu = (uint32_t)acc[4 * HF + (q >> 2)][j][q & 3] - (uint32_t)czab[q];
                    if (a.b_zp) {  // weight zero points (rare): per-column terms read here
                        const int nn = min(nc0 + q, a.N - 1);
                        const uint32_t zb = (uint32_t)(int)a.b_zp[nn];
                        accu -= zb * (uint32_t)asum;
                        accu += (uint32_t)a.K * (uint32_t)p.za * zb;
                    }
                    if (INT_CODES) {
                        const float sc = rsa[j] * csb[q];
                        float y = (float)(int32_t)accu * sc;
                        if (BIAS) y = y + cbias[q];
                        if (RELU) y = (y <= 0.0f) ? 0.0f : y;
                        out[q] = (uint32_t)requant_int<KIND>(y, p, cc);
                        if (KIND == LQ_OUT_QU8S8) out[q] ^= 0x80u;
                    } else {
                        out[q] = epi_one<KIND>((int32_t)accu, rsa[j], csb[q], BIAS ? &cbias[q] : nullptr, RELU, p,
                                               a.gelu != 0);
                    }
                }
                if constexpr (KIND == LQ_OUT_F32) {
                    if (a.extrema && m < a.M) {
#pragma unroll
                        for (int q = 0; q < 16; ++q)
                            if (nc0 + q < a.N) key_accum(ext_min, ext_max, __uint_as_float(out[q]));
                    }
                }
                store_row(j, out);
            });
        };
        if (has_bias) {
            if (relu) rows_general(std::true_type{}, std::true_type{});
            else rows_general(std::true_type{}, std::false_type{});
        } else {
            if (relu) rows_general(std::false_type{}, std::true_type{});
            else rows_general(std::false_type{}, std::false_type{});
        }
    };
    epilogue_half(std::integral_constant<int, 0>());
    if constexpr (NH > 1) epilogue_half(std::integral_constant<int, 1>());
    if constexpr (KIND == LQ_OUT_F32) {
        if (a.extrema) {  // the workgroup's pair of keys, for a dynamic quantize of the output
            __shared__ int32_t emin[NW], emax[NW];
            ext_min = wave_min(ext_min);
            ext_max = wave_max(ext_max);
            if (lane == 0) {
                emin[wave] = ext_min;
                emax[wave] = ext_max;
            }
            __syncthreads();
            if (threadIdx.x == 0) {
                for (int w = 1; w < NW; ++w) {
                    ext_min = min(ext_min, emin[w]);
                    ext_max = max(ext_max, emax[w]);
                }
                a.extrema[blockIdx.x] = make_int2(ext_min, ext_max);
            }
        }
    }
}

// ------------------------------------------------------ skinny-M (decode) kernel
//
// M <= 16*MT.  One workgroup owns 16 output columns n and all M rows; its W waves split K
// into W contiguous ranges and stream their share of the 16 B rows straight from HBM into
// MFMA registers (every B byte is read once), UNROLL k-steps of 64 in flight per wave.
// A (M x K, a few KB) stays L2-resident.  Partial accumulators are summed through LDS.

template <int MT, int W, int KIND, int UNROLL = 8>
__global__ __launch_bounds__(64 * W) void gemm_i8_skinny_kernel(GemmArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * 16;
    const int nrow = n0 + (lane & 15);
    const int kg = (lane >> 4) * 16;

    const int ksteps = (a.K + 63) / 64;
    const int per_wave = (ksteps + W - 1) / W;
    const int ks_begin = wave * per_wave;
    const int ks_end = min(ksteps, ks_begin + per_wave);

    v4i acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = v4i{0, 0, 0, 0};

    const int8_t* brow = a.B + (int64_t)nrow * a.ldb;
    const bool nrow_ok = nrow < a.N;
    for (int ks = ks_begin; ks < ks_end; ks += UNROLL) {
        v4i bf[UNROLL], af[UNROLL][MT];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int k = (ks + u) * 64 + kg;
            const bool ok = (ks + u < ks_end) && k < a.K;
            bf[u] = (ok && nrow_ok) ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(brow + k))
                                    : v4i{0, 0, 0, 0};
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const int m = t * 16 + (lane & 15);
                af[u][t] = (ok && m < a.M) ? *reinterpret_cast<const v4i*>(a.A + (int64_t)m * a.lda + k)
                                           : v4i{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u)
#pragma unroll
            for (int t = 0; t < MT; ++t)
                acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[u], af[u][t], acc[t], 0, 0, 0);
    }

    const EpiParams p = epi_params(a);
    if (W > 1) {
        // the waves' partial sums meet in LDS; wave w then adds up (in wave order) and stores
        // the m-tiles t = w, w + W, ...
        __shared__ v4i red[W][MT][64];
#pragma unroll
        for (int t = 0; t < MT; ++t) red[wave][t][lane] = acc[t];
        __syncthreads();
        for (int t = wave; t < MT; t += W) {
            v4i s = red[0][t][lane];
            for (int w = 1; w < W; ++w) s += red[w][t][lane];
            epilogue4<KIND>(a, p, t * 16 + (lane & 15), n0 + (lane >> 4) * 4, s);
        }
        return;
    }

    static_for<MT>([&](auto t_c) __attribute__((always_inline)) {
        constexpr int t = decltype(t_c)::value;
        const int m = t * 16 + (lane & 15);
        const int n = n0 + (lane >> 4) * 4;
        epilogue4<KIND>(a, p, m, n, acc[t]);
    });
}

// --------------------------------------------- packed weights (decode, M <= 64)
//
// MFMA-packed weight layout: B [N, K] int8 cut into tiles of 16 rows x 64 K-bytes; tile
// (t, s) occupies bytes [(t * KS + s) * 1024, +1024) with KS = ceil(K / 64), and its lane-l
// 16-byte chunk holds row 16 t + l % 16, K-bytes 64 s + 16 (l / 16) .. +15: exactly the
// A-operand fragment of v_mfma_i32_16x16x64_i8.  Rows past N and bytes past K are zero.
// One wave load is then 1 KB contiguous, where a row-major weight gives 16 rows x 64 bytes.

constexpr int PACK_TILE = 1024;

__global__ __launch_bounds__(256) void pack_weights_i8_kernel(const int8_t* __restrict__ B, int64_t ldb, int N,
                                                              int K, int KS, int64_t chunks,
                                                              int8_t* __restrict__ P) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= chunks) return;
    const int l = (int)(c & 63);
    const int64_t tile = c >> 6;
    const int t = (int)(tile / KS), s = (int)(tile % KS);
    const int row = t * 16 + (l & 15);
    const int k0 = s * 64 + (l >> 4) * 16;
    int8_t v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = (row < N && k0 + j < K) ? B[(int64_t)row * ldb + k0 + j] : (int8_t)0;
    *reinterpret_cast<v4i*>(P + c * 16) = *reinterpret_cast<const v4i*>(v);
}

// One workgroup per 16-row n-tile, its W waves splitting the K steps; every tile byte is
// read once, UNROLL steps (16 KB per wave) in flight.  A (M x K, a few KB) stays in L2.
template <int MT, int W, int UNROLL, int KIND>
__global__ __launch_bounds__(64 * W) void gemm_i8_packed_skinny_kernel(GemmArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x;
    const int KS = (a.K + 63) / 64;
    const int per = (KS + W - 1) / W;
    const int kb = wave * per, ke = min(KS, kb + per);
    const int kg = (lane >> 4) * 16;
    v4i acc[MT];
#pragma unroll
    for (int u = 0; u < MT; ++u) acc[u] = v4i{0, 0, 0, 0};
    const int8_t* bt = a.B + (int64_t)t * KS * PACK_TILE + lane * 16;
    for (int ks = kb; ks < ke; ks += UNROLL) {
        v4i bf[UNROLL], af[UNROLL][MT];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const bool ok = ks + u < ke;
            const int k = (ks + u) * 64 + kg;
            bf[u] = ok ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(bt + (int64_t)(ks + u) * PACK_TILE))
                       : v4i{0, 0, 0, 0};
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int m = mt * 16 + (lane & 15);
                af[u][mt] = (ok && k < a.K && m < a.M) ? *reinterpret_cast<const v4i*>(a.A + (int64_t)m * a.lda + k)
                                                       : v4i{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                acc[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[u], af[u][mt], acc[mt], 0, 0, 0);
    }
    __shared__ v4i red[W][MT][64];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[wave][mt][lane] = acc[mt];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        v4i sum = red[0][mt][lane];
        for (int w = 1; w < W; ++w) sum += red[w][mt][lane];
        acc[mt] = sum;
    }
    const EpiParams p = epi_params(a);
    const int n = t * 16 + (lane >> 4) * 4;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) epilogue4<KIND>(a, p, mt * 16 + (lane & 15), n, acc[mt]);
}

// ----------------------------------------- packed weights, 64 < M <= 128 (decode)
//
// The skinny kernel above keeps A's fragments in registers next to the weight stream; at
// M = 128 that leaves room for two 1 KB weight loads in flight per wave and re-reads all of
// A per 16 columns, so it waits on latency.  Here a workgroup owns 64 columns (one 16-column
// n-tile per wave) and one K-split (gridDim.y): the split's A slice (M rows x up to 1 KB) is
// staged once in LDS and shared by the four waves, and each wave issues every weight k-step
// of its split at once (up to 16 KB in flight).  Chunk c of A row r sits at chunk slot
// c ^ (r % 16) of the row, so the 16 rows a fragment read touches fall in 16 different bank
// groups.  Each split stores its exact int32 partial sums to the workspace
// ([split][m][n], rows padded to whole n-tiles); gemm_i8_decode_reduce_kernel adds the splits
// in order and runs the epilogue.

constexpr int DEC_MAX_KS = 16;  // k-steps (64 B) per split at most: a 1 KB A row slice (M = 128: 128 KB of LDS)

struct DecodePlan {
    int ks_per_split, splits;
    int64_t npad;  // partial row pitch (whole 16-column n-tiles)
};

static DecodePlan decode_plan(int64_t M, int64_t N, int64_t K) {
    (void)M;
    DecodePlan p;
    const int64_t KS = (K + 63) / 64, tiles64 = (N + 63) / 64;
    p.ks_per_split = DEC_MAX_KS;
    p.splits = (int)((KS + p.ks_per_split - 1) / p.ks_per_split);
    // at least 256 workgroups when K allows (whole groups of 4 k-steps per split)
    while (tiles64 * p.splits < 256 && p.ks_per_split > 4) {
        p.ks_per_split -= 4;
        p.splits = (int)((KS + p.ks_per_split - 1) / p.ks_per_split);
    }
    if (p.splits < 1) p.splits = 1;
    p.npad = (N + 15) / 16 * 16;
    return p;
}

// M from which the packed path takes the split-K decode kernel (below it the skinny kernel,
// whose per-16-column re-read of A is small).
constexpr int DEC_MIN_M = 33;

static size_t decode_partial_bytes(int64_t M, int64_t N, int64_t K) {
    if (M < DEC_MIN_M || M > 128) return 0;
    const DecodePlan p = decode_plan(M, N, K);
    return sizeof(int32_t) * (size_t)p.splits * (size_t)M * (size_t)p.npad;
}

template <int MT>
__global__ __launch_bounds__(256) void gemm_i8_decode_partial_kernel(GemmArgs a, int ks_per_split, int64_t npad,
                                                                      int32_t* __restrict__ part) {
    __shared__ __attribute__((aligned(1024))) int8_t As[MT * 16 * DEC_MAX_KS * 64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int KS = (a.K + 63) / 64;
    const int split = blockIdx.y;
    const int ks0 = split * ks_per_split, nks = min(KS - ks0, ks_per_split);  // >= 1 by the plan
    const int slots = ks_per_split * 4;  // 16-byte chunk slots per A row in LDS (a multiple of 16)
    // This wave's share of the A slice goes straight into LDS first, then its weight k-steps
    // (exactly DEC_MAX_KS loads, steps past the split clamped to its last): vmcnt counts both
    // in issue order, so vmcnt(DEC_MAX_KS) means this wave's A copies have landed while the
    // weights are still streaming, and each k-step below starts as soon as its weight is in.
    // A slice: MT*16 rows x `slots` chunks, copied 64 chunks (1 KB) per wave instruction.
    // LDS slot g = row * slots + s holds global chunk c = s ^ (row % 16) of the row (rows
    // past M read as zeros through the buffer bound; chunks past the split's K are never read).
    const v4i ra = buffer_rsrc(a.A, (uint32_t)((int64_t)a.M * a.lda));
    const uint32_t lds_base = (uint32_t)reinterpret_cast<uintptr_t>(As);
    const int copies = MT * 16 * slots / 64;
    for (int q = wave; q < copies; q += 4) {
        const int g = q * 64 + lane, r = g / slots, sl = g - r * slots;
        const uint32_t voff = (uint32_t)r * (uint32_t)a.lda + (uint32_t)((ks0 * 4 + (sl ^ (r & 15))) * 16);
        lds_dma16(ra, voff, 0u, lds_base + (uint32_t)q * 1024u);
    }
    const int t = blockIdx.x * 4 + wave;  // this wave's 16-column n-tile
    const bool has_tile = t * 16 < a.N;
    const int tc = has_tile ? t : 0;      // a valid tile to read when this wave has none
    const int8_t* bt = a.B + ((int64_t)tc * KS + ks0) * PACK_TILE + lane * 16;
    v4i bf[DEC_MAX_KS];
#pragma unroll
    for (int j = 0; j < DEC_MAX_KS; ++j)
        bf[j] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(bt + (int64_t)min(j, nks - 1) * PACK_TILE));
    wait_vmcnt<DEC_MAX_KS>();
    block_barrier();  // every wave's A copies have landed (no fence: the weights keep streaming)
    if (!has_tile) {
        wait_vmcnt<0>();  // no load may be in flight when the wave ends
        return;
    }
    v4i acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = v4i{0, 0, 0, 0};
    const int rl = lane & 15, cq = lane >> 4;
#pragma unroll
    for (int j = 0; j < DEC_MAX_KS; ++j) {
        if (j < nks) {  // wave-uniform; a predicate, not a break, keeps bf[] in registers
            const int c = j * 4 + cq;
            v4i af[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int r = mt * 16 + rl;
                af[mt] = *reinterpret_cast<const v4i*>(As + (r * slots + (c ^ (r & 15))) * 16);
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                acc[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[j], af[mt], acc[mt], 0, 0, 0);
        }
    }
    // lane l holds C[m = 16 mt + l % 16][n = 16 t + 4 (l / 16) .. +3]
    const int n = t * 16 + cq * 4;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + rl;
        if (m < a.M) *reinterpret_cast<v4i*>(part + ((int64_t)split * a.M + m) * npad + n) = acc[mt];
    }
}

template <int KIND>
__global__ __launch_bounds__(256) void gemm_i8_decode_reduce_kernel(GemmArgs a, int splits, int64_t npad,
                                                                     const int32_t* __restrict__ part) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;  // one quad of 4 columns
    const int64_t quads = npad / 4;
    if (q >= (int64_t)a.M * quads) return;
    const int m = (int)(q / quads), n = (int)(q - (int64_t)m * quads) * 4;
    if (n >= a.N) return;
    // the epilogue's inputs are loaded with the partial sums, not after them (one round trip)
    const EpiParams p = epi_params(a);
    const RowCtx row = load_row(a, m);
    const ColCtx cols = load_cols<KIND>(a, n);
    // U splits' loads in flight at a time, none past the last split (integer sums: exact in
    // any order)
    v4i acc = v4i{0, 0, 0, 0};
    auto add_splits = [&](auto uc) {
        constexpr int U = decltype(uc)::value;
        for (int s0 = 0; s0 < splits; s0 += U) {
            v4i v[U];
#pragma unroll
            for (int u = 0; u < U; ++u)
                v[u] = s0 + u < splits ? *reinterpret_cast<const v4i*>(part + ((int64_t)(s0 + u) * a.M + m) * npad + n)
                                       : v4i{0, 0, 0, 0};
#pragma unroll
            for (int u = 0; u < U; ++u) acc += v[u];
        }
    };
    if (splits <= 4) add_splits(std::integral_constant<int, 4>());
    else add_splits(std::integral_constant<int, 8>());
    epilogue4c<KIND>(a, p, row, cols, m, acc);
}

template <int KIND>
static int launch_packed_skinny(const GemmArgs& a, hipStream_t st) {
    const unsigned tiles = (unsigned)((a.N + 15) / 16);
    if (a.M <= 16)
        hipLaunchKernelGGL((gemm_i8_packed_skinny_kernel<1, 4, 16, KIND>), dim3(tiles), dim3(256), 0, st, a);
    else if (a.partial != nullptr) {
        const DecodePlan p = decode_plan(a.M, a.N, a.K);
        const dim3 grid((unsigned)((a.N + 63) / 64), (unsigned)p.splits);
        if (a.M <= 32)
            hipLaunchKernelGGL((gemm_i8_decode_partial_kernel<2>), grid, dim3(256), 0, st, a, p.ks_per_split, p.npad,
                               a.partial);
        else if (a.M <= 64)
            hipLaunchKernelGGL((gemm_i8_decode_partial_kernel<4>), grid, dim3(256), 0, st, a, p.ks_per_split, p.npad,
                               a.partial);
        else
            hipLaunchKernelGGL((gemm_i8_decode_partial_kernel<8>), grid, dim3(256), 0, st, a, p.ks_per_split, p.npad,
                               a.partial);
        const int64_t quads = (int64_t)a.M * (p.npad / 4);
        hipLaunchKernelGGL((gemm_i8_decode_reduce_kernel<KIND>), dim3((unsigned)((quads + 255) / 256)), dim3(256), 0,
                           st, a, p.splits, p.npad, a.partial);
        note_path(a.M <= 32 ? "gemm packed decode m32 split-k" : a.M <= 64 ? "gemm packed decode m64 split-k"
                            : "gemm packed decode m128 split-k");
        return launch_status("lq_gemm_w8a8_packed (decode)");
    } else if (a.M <= 32)
        hipLaunchKernelGGL((gemm_i8_packed_skinny_kernel<2, 4, 8, KIND>), dim3(tiles), dim3(256), 0, st, a);
    else if (a.M <= 64)
        hipLaunchKernelGGL((gemm_i8_packed_skinny_kernel<4, 4, 4, KIND>), dim3(tiles), dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((gemm_i8_packed_skinny_kernel<8, 4, 2, KIND>), dim3(tiles), dim3(256), 0, st, a);
    note_path(a.M <= 16 ? "gemm packed skinny m16" : a.M <= 32 ? "gemm packed skinny m32"
              : a.M <= 64 ? "gemm packed skinny m64" : "gemm packed skinny m128");
    return launch_status("lq_gemm_w8a8_packed");
}

// ------------------------------------------ dynamic Linear at decode sizes, one launch
//
// nnqd.Linear's forward for M <= 16 rows in one launch (lq_dynamic_linear_packed_f32).  The
// launches it replaces -- the layer norm of the float module before it (after its residual
// add), lq_dynamic_quantize_f32 (live min / max, per-tensor affine qparams, codes c - 128)
// and lq_gemm_w8a8_packed -- each wait for the one before, and at decode sizes each is a few
// microseconds of latency around little work.  Here every workgroup builds the whole int8
// input itself, in LDS: at most 16 rows, re-read from L2 by each workgroup, while the weight
// -- the bytes that count -- is still read once.  A workgroup issues its first weight loads
// before the input work, so their latency runs under it.  The norm is ln_row (the order of
// the standalone norm), the extrema are order-free, the qparams and codes are dyn_qparams and
// quant_one with the same reciprocal, and the products are exact int32 sums: the launches'
// bits.
//
// WT: each of the 4 waves owns a 16-column tile and all of K (wide N, so fewer workgroups
// repeat the input work); otherwise the waves split the K steps of one tile and meet in LDS
// (gemm_i8_packed_skinny_kernel's split).
enum { DL_PLAIN = 0, DL_LN = 1, DL_ADD_LN = 2 };  // LQ_DL_*
constexpr int DL_MAX_MK = 16384;                   // input values (held in registers, 16 x 4 per lane)
constexpr int DL_MAX_MK_LN = 8192;                 // normalized values staged in LDS (32 KB)
constexpr int DL_MAX_K_LN = 32 * LN_T;             // row width ln_load<8> keeps in registers
constexpr int DL_UNROLL = 8;
constexpr int64_t DL_WT_MIN_TILES = 512;  // from here on, wave tiles (N >= 8192)

struct DynLinArgs {
    const float* x;
    int64_t ldx;
    const float* res;  // DL_ADD_LN
    int64_t ldres;
    float* sum;  // x + res out (workgroup 0), or null; never x itself (other workgroups read x)
    int64_t ldsum;
    const float* gamma;
    const float* beta;
    float ln_eps;
    int qmin;
    float eps, width_f;
    Grid g;
    float* qp;  // {min, max, scale, zero point} out (workgroup 0), or null
    int KP;     // LDS row stride of the codes: the K steps' bytes + 16 (16 rows on distinct banks)
};

// Codes c - 128 of four values as one dword (byte e = value e).
// (quant_store: the integer-domain form of Code::store(quant_one(...)), the same codes)
__device__ __forceinline__ uint32_t dl_codes4(vf4 v, float inv, float z, const Grid& g) {
    const uint32_t c0 = (uint8_t)quant_store<CodeU8S8>(v.x, inv, z, g);
    const uint32_t c1 = (uint8_t)quant_store<CodeU8S8>(v.y, inv, z, g);
    const uint32_t c2 = (uint8_t)quant_store<CodeU8S8>(v.z, inv, z, g);
    const uint32_t c3 = (uint8_t)quant_store<CodeU8S8>(v.w, inv, z, g);
    return c0 | (c1 << 8) | (c2 << 16) | (c3 << 24);
}

// MAXC: chunks per lane of a normalized row; RPW: rows per wave (M <= 4 RPW); both unused by
// DL_PLAIN, whose M x K values stay in registers (16 float4 per lane).
template <int SRC, bool WT, int MAXC, int RPW, int KIND>
__global__ __launch_bounds__(256) void dyn_linear_skinny_kernel(DynLinArgs d, GemmArgs a) {
    extern __shared__ __align__(16) uint8_t dl_lds[];
    __shared__ int32_t smin[4], smax[4];
    __shared__ v4i red[WT ? 1 : 4][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int M = a.M, K = a.K, KS = (K + 63) / 64, tiles = (a.N + 15) / 16;
    int8_t* cs = reinterpret_cast<int8_t*>(dl_lds);  // codes c - 128, [M][KP]
    float* ys = reinterpret_cast<float*>(dl_lds + ((M * d.KP + 15) & ~15));  // normalized rows [M][K]

    // ---- everything that does not depend on the input, in flight first: this wave's first
    // weight steps and its output columns' epilogue inputs
    const int tile = WT ? blockIdx.x * 4 + wave : blockIdx.x;
    const int per = WT ? KS : (KS + 3) / 4;
    const int kb = WT ? 0 : wave * per, ke = min(KS, kb + per);
    const int8_t* bt = a.B + (int64_t)min(tile, tiles - 1) * KS * PACK_TILE + lane * 16;
    v4i bf[DL_UNROLL];
#pragma unroll
    for (int u = 0; u < DL_UNROLL; ++u)
        bf[u] = kb + u < ke ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(bt + (int64_t)(kb + u) * PACK_TILE))
                            : v4i{0, 0, 0, 0};
    // the column inputs as loaded values only (a conversion here would wait for the weights):
    // symmetric weights, no zero-point column
    const int n = min(tile, tiles - 1) * 16 + (lane >> 4) * 4;
    ColCtx cols;
    cols.n = n;
    cols.vec = vec_store_ok(a, n, OutTraits<KIND>::bytes);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int nn = min(n + r, a.N - 1);
        cols.sb[r] = a.b_scale[nn];
        cols.bias[r] = a.bias ? a.bias[nn] : 0.0f;
        cols.bsum[r] = a.b_sums[nn];
        cols.zb[r] = 0;
    }

    // ---- the input values and the keys of their extrema
    int32_t kmin = KEY_POS_INF, kmax = KEY_NEG_INF;
    const int K4 = K >> 2;
    constexpr int XV = DL_MAX_MK / (4 * 256);
    vf4 xv[SRC == DL_PLAIN ? XV : 1];
    if constexpr (SRC == DL_PLAIN) {
#pragma unroll
        for (int j = 0; j < XV; ++j) {
            const int i = tid + 256 * j;
            if (i < M * K4) {
                const int r = i / K4;
                xv[j] = *reinterpret_cast<const vf4*>(d.x + (int64_t)r * d.ldx + 4 * (i - r * K4));
            }
        }
#pragma unroll
        for (int j = 0; j < XV; ++j)
            if (tid + 256 * j < M * K4) {
                key_accum(kmin, kmax, xv[j].x);
                key_accum(kmin, kmax, xv[j].y);
                key_accum(kmin, kmax, xv[j].z);
                key_accum(kmin, kmax, xv[j].w);
            }
    } else {
        // rows wave, wave + 4, ...: every row of the wave loaded before any is normalized
        float v[RPW][4 * MAXC], rv[RPW][4 * MAXC];
#pragma unroll
        for (int q = 0; q < RPW; ++q) {
            const int r = wave + 4 * q;
            const bool act = r < M;
            const int rc = act ? r : 0;
            ln_fetch<MAXC>(d.x + (int64_t)rc * d.ldx, SRC == DL_ADD_LN ? d.res + (int64_t)rc * d.ldres : nullptr, act,
                           K, lane, v[q], rv[q]);
        }
#pragma unroll
        for (int q = 0; q < RPW; ++q) {
            const int r = wave + 4 * q;
            const bool act = r < M;
            float* wb = (SRC == DL_ADD_LN && d.sum && blockIdx.x == 0) ? d.sum + (int64_t)(act ? r : 0) * d.ldsum
                                                                        : nullptr;
            ln_add_store<MAXC>(v[q], rv[q], SRC == DL_ADD_LN, wb, act, K, lane);
        }
#pragma unroll
        for (int q = 0; q < RPW; ++q) {
            const int r = wave + 4 * q;
            if (r >= M) continue;  // the whole wave: no row
            ln_norm<MAXC>(v[q], true, K, lane, d.gamma, d.beta, d.ln_eps, ys + r * K);
            {
#pragma unroll
                for (int j = 0; j < MAXC; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (4 * (lane + LN_T * j) + e < K) key_accum(kmin, kmax, v[q][4 * j + e]);
            }
        }
    }
    kmin = wave_min(kmin);
    kmax = wave_max(kmax);
    if (lane == 0) {
        smin[wave] = kmin;
        smax[wave] = kmax;
    }
    __syncthreads();  // also publishes ys
    kmin = min(min(smin[0], smin[1]), min(smin[2], smin[3]));
    kmax = max(max(smax[0], smax[1]), max(smax[2], smax[3]));
    float o[4];
    dyn_qparams(kmin, kmax, d.qmin, d.eps, d.width_f, d.g, o);
    const float sc = o[2], z = o[3];
    const float inv = 1.0f / sc;
    if (d.qp && blockIdx.x == 0 && tid == 0) {
        d.qp[0] = o[0];
        d.qp[1] = o[1];
        d.qp[2] = o[2];
        d.qp[3] = o[3];
    }

    // ---- the codes, row-major in LDS with a zero tail up to whole K steps
    if constexpr (SRC == DL_PLAIN) {
#pragma unroll
        for (int j = 0; j < XV; ++j) {
            const int i = tid + 256 * j;
            if (i < M * K4) {
                const int r = i / K4, k = 4 * (i - r * K4);
                *reinterpret_cast<uint32_t*>(cs + r * d.KP + k) = dl_codes4(xv[j], inv, z, d.g);
            }
        }
    } else {
        for (int i = tid; i < M * K4; i += 256) {
            const int r = i / K4, k = 4 * (i - r * K4);
            *reinterpret_cast<uint32_t*>(cs + r * d.KP + k) =
                dl_codes4(*reinterpret_cast<const vf4*>(ys + r * K + k), inv, z, d.g);
        }
    }
    const int tail4 = (KS * 64 - K) >> 2;
    for (int i = tid; i < M * tail4; i += 256) {
        const int r = i / tail4;
        *reinterpret_cast<uint32_t*>(cs + r * d.KP + K + 4 * (i - r * tail4)) = 0u;
    }
    __syncthreads();

    // ---- the product: weights from registers, code fragments from LDS (rows past M read the
    // last row; their outputs are never stored)
    const int8_t* arow = cs + min(lane & 15, M - 1) * d.KP + (lane >> 4) * 16;
    v4i acc = v4i{0, 0, 0, 0};
    for (int ks = kb; ks < ke; ks += DL_UNROLL) {
#pragma unroll
        for (int u = 0; u < DL_UNROLL; ++u)
            if (ks + u < ke)
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[u], *reinterpret_cast<const v4i*>(arow + (ks + u) * 64),
                                                            acc, 0, 0, 0);
        if (ks + DL_UNROLL < ke) {
#pragma unroll
            for (int u = 0; u < DL_UNROLL; ++u) {
                const int k2 = ks + DL_UNROLL + u;
                bf[u] = k2 < ke ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(bt + (int64_t)k2 * PACK_TILE))
                                : v4i{0, 0, 0, 0};
            }
        }
    }
    if constexpr (!WT) {
        red[wave][lane] = acc;
        __syncthreads();
        if (wave != 0) return;
        acc = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
    }
    if (tile >= tiles) return;
    EpiParams p = epi_params(a);
    p.za = (int)z - 128;  // the codes' zero point, in the stored c - 128 units
    p.has_za = true;
    RowCtx row;
    row.sa = sc;
    row.asum = 0;
    epilogue4c<KIND>(a, p, row, cols, lane & 15, acc);
}

// ------------------------------------------------------------ generic kernel
// Any K, alignment and leading dimensions (byte loads, dot4 on the fly): the fallback for
// shapes the vector paths do not take.  One thread per output.
template <int KIND>
__global__ __launch_bounds__(256) void gemm_i8_generic_kernel(GemmArgs a) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)a.M * a.N) return;
    const int m = (int)(idx / a.N), n = (int)(idx % a.N);
    const int8_t* ar = a.A + (int64_t)m * a.lda;
    const int8_t* br = a.B + (int64_t)n * a.ldb;
    uint32_t s = 0;
    for (int k = 0; k < a.K; ++k) s += (uint32_t)((int)ar[k] * (int)br[k]);
    const EpiParams p = epi_params(a);
    int32_t acc = corrected((int32_t)s, m, n, a, p);
    const float sa = a.a_scale ? a.a_scale[(int64_t)m * a.a_stride] : 1.0f;
    const float sb = a.b_scale ? a.b_scale[(int64_t)n * a.b_stride] : 1.0f;
    store_elem<KIND>(a.C, (int64_t)m * a.ldc + n,
                     epi_one<KIND>(acc, sa, sb, a.bias ? a.bias + n : nullptr, a.relu != 0, p, a.gelu != 0));
}

// ------------------------------------------------------------------ row sums
// sums[r] = sum_k X[r,k] (int8), one wave per row.
__global__ __launch_bounds__(256) void row_sums_i8_kernel(const int8_t* __restrict__ X, int64_t ld,
                                                          int64_t rows, int64_t K,
                                                          int32_t* __restrict__ sums) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const int8_t* x = X + r * ld;
    int s = 0;
    for (int64_t k = lane; k < K; k += 64) s += x[k];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) sums[r] = s;
}

// ------------------------------------------------------------------- dispatch

// With a.extrema (float32 out): only the LDS-DMA kernels fold their output's extrema, into at
// most DYN_PARTS_MAX pairs; any other route returns LQ_ERR_UNSUPPORTED before launching
// anything (the caller then runs the product and the dynamic quantize as separate calls), and
// *ext_parts receives the number of pairs written.
constexpr int GEMM_NO_EXTREMA = LQ_ERR_UNSUPPORTED;

template <int KIND>
struct GemmLaunch {
    static int run(const GemmArgs& a0, hipStream_t st, int64_t workspace_split_bytes, int* ext_parts = nullptr) {
        GemmArgs a = a0;
        const bool vec = aligned16(a.A) && aligned16(a.B) && (a.lda % 16 == 0) && (a.ldb % 16 == 0) &&
                         (a.K % 16 == 0);
        const bool dma_ok = (a.K % 128 == 0) && ((int64_t)(a.M + 256) * a.lda < (int64_t)1 << 31) &&
                            ((int64_t)(a.N + 256) * a.ldb < (int64_t)1 << 31);
        const int64_t tiles128 = ((int64_t)(a.M + 127) / 128) * ((a.N + 127) / 128);
        if (a.extrema) {
            // the route must be one of the DMA kernels below, with few enough workgroups
            if (KIND != LQ_OUT_F32 || !vec || a.M <= 64 || (a.M <= 128 && tiles128 < 128) || !dma_ok ||
                tiles128 < 128 || tiles128 > DYN_PARTS_MAX)
                return GEMM_NO_EXTREMA;
        }
        if (!vec) {
            const int64_t total = (int64_t)a.M * a.N;
            hipLaunchKernelGGL(gemm_i8_generic_kernel<KIND>, dim3((unsigned)((total + 255) / 256)),
                               dim3(256), 0, st, a);
            note_path("gemm generic");
            return launch_status("lq_gemm_w8a8 (generic)");
        }
        if (a.M <= 16) {
            hipLaunchKernelGGL((gemm_i8_skinny_kernel<1, 8, KIND>), dim3((unsigned)((a.N + 15) / 16)),
                               dim3(512), 0, st, a);
            note_path("gemm skinny");
            return launch_status("lq_gemm_w8a8 (skinny)");
        }
        if (a.M <= 32) {
            hipLaunchKernelGGL((gemm_i8_skinny_kernel<2, 8, KIND>), dim3((unsigned)((a.N + 15) / 16)),
                               dim3(512), 0, st, a);
            note_path("gemm skinny");
            return launch_status("lq_gemm_w8a8 (skinny)");
        }
        if (a.M <= 64) {
            hipLaunchKernelGGL((gemm_i8_skinny_kernel<4, 8, KIND>), dim3((unsigned)((a.N + 15) / 16)),
                               dim3(512), 0, st, a);
            note_path("gemm skinny");
            return launch_status("lq_gemm_w8a8 (skinny)");
        }
        if (a.M <= 128 && tiles128 < 128) {
            hipLaunchKernelGGL((gemm_i8_skinny_kernel<8, 8, KIND, 2>), dim3((unsigned)((a.N + 15) / 16)),
                               dim3(512), 0, st, a);
            note_path("gemm skinny");
            return launch_status("lq_gemm_w8a8 (skinny)");
        }
        // LDS-DMA path: whole 128-byte K stages, 32-bit buffer offsets (dma_ok above).
        const int64_t dma_tiles = ((int64_t)(a.M + 255) / 256) * ((a.N + 127) / 128);
        // 256x256 tiles (8 waves of 128x64: a third fewer LDS fragment bytes per MFMA) take
        // ~15% less time per op than 256x128 tiles (waves of 64x64) but come in half as many
        // workgroups: compare the two in rounds of 256 workgroups (one per CU).
        const int64_t t256 = ((int64_t)(a.M + 255) / 256) * ((a.N + 255) / 256);
        if (dma_ok && t256 >= 256 && ((t256 + 255) / 256) * 100 <= ((dma_tiles + 255) / 256) * 57) {
            if (ext_parts) *ext_parts = (int)t256;
            hipLaunchKernelGGL((gemm_i8_dma_kernel<256, 256, 2, 4, GEMM_NBUF, KIND>), dim3((unsigned)t256),
                               dim3(512), 0, st, a);
            note_path("gemm dma 256x256");
            return launch_status("lq_gemm_w8a8 (dma 256x256)");
        }
        if (dma_ok && dma_tiles >= 256) {
            if (ext_parts) *ext_parts = (int)dma_tiles;
            hipLaunchKernelGGL((gemm_i8_dma_kernel<256, 128, 4, 2, GEMM_NBUF, KIND>), dim3((unsigned)dma_tiles),
                               dim3(512), 0, st, a);
            note_path("gemm dma 256x128");
            return launch_status("lq_gemm_w8a8 (dma 256x128)");
        }
        const int64_t dma_tiles_128 = ((int64_t)(a.M + 127) / 128) * ((a.N + 127) / 128);
        if (dma_ok && dma_tiles_128 >= 128) {
            if (ext_parts) *ext_parts = (int)dma_tiles_128;
            // One round of tiles (at most one per CU): the LDS a second workgroup per CU would
            // use goes to a third ring stage (M = 1024, N = K = 4096: 26.6 -> 20.8 us; a fourth
            // stage, or the K stages split between two wave groups of 8 waves, no better).  At
            // most half a round: 128x64 tiles of four waves with four-stage rings, twice the
            // workgroups (M = 512, N = K = 4096: 16.7 -> 14.3 us).
            if (dma_tiles_128 <= 128) {
                const int64_t tiles64 = ((int64_t)(a.M + 127) / 128) * ((a.N + 63) / 64);
                if (ext_parts) *ext_parts = (int)tiles64;
                hipLaunchKernelGGL((gemm_i8_dma_kernel<128, 64, 4, 1, 4, KIND>), dim3((unsigned)tiles64),
                                   dim3(256), 0, st, a);
                note_path("gemm dma 128x64");
                return launch_status("lq_gemm_w8a8 (dma 128x64)");
            }
            if (dma_tiles_128 <= 256) {
                hipLaunchKernelGGL((gemm_i8_dma_kernel<128, 128, 4, 2, 3, KIND>), dim3((unsigned)dma_tiles_128),
                                   dim3(512), 0, st, a);
                note_path("gemm dma 128x128 3-stage");
                return launch_status("lq_gemm_w8a8 (dma 128x128 3-stage)");
            }
            hipLaunchKernelGGL((gemm_i8_dma_kernel<128, 128, 4, 2, GEMM_NBUF, KIND>), dim3((unsigned)dma_tiles_128),
                               dim3(512), 0, st, a);
            note_path("gemm dma 128x128");
            return launch_status("lq_gemm_w8a8 (dma 128x128)");
        }
        const int64_t mid_tiles = ((int64_t)(a.M + 127) / 128) * ((a.N + 127) / 128);
        int splits = 1;
        const int nk = (a.K + BK - 1) / BK;
        if (mid_tiles < 256 && workspace_split_bytes > 0) {
            splits = (int)((256 + mid_tiles - 1) / mid_tiles);
            if (splits > nk / 4) splits = nk / 4;  // keep at least 4 stages per split
            if (splits < 1) splits = 1;
        }
        a.splits = splits;
        if (splits > 1) {
            int rc = lq_fill_u32(a.partial, 0u, (size_t)a.M * a.N, st);
            if (rc) return rc;
            rc = lq_fill_u32(a.counters, 0u, (size_t)mid_tiles, st);
            if (rc) return rc;
        }
        hipLaunchKernelGGL((gemm_i8_tiled_kernel<128, 128, 2, 2, KIND>),
                           dim3((unsigned)(mid_tiles * splits)), dim3(256), 0, st, a);
        note_path(splits > 1 ? "gemm 128x128 split-k" : "gemm 128x128");
        return launch_status("lq_gemm_w8a8 (128x128)");
    }
};

static bool valid_out_kind(int k) { return k >= LQ_OUT_I32 && k <= LQ_OUT_QU8S8; }

// Workspace layout: [a_sums M][b_sums N][split partial M*N][tile counters], 256-byte aligned parts.
struct GemmWs {
    size_t a_sums, b_sums, partial, counters, total;
};
static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
static GemmWs gemm_ws(int64_t M, int64_t N, int64_t K) {
    GemmWs w;
    w.a_sums = 0;
    w.b_sums = w.a_sums + align256(sizeof(int32_t) * (size_t)M);
    w.partial = w.b_sums + align256(sizeof(int32_t) * (size_t)N);
    // split-K partials: the row-major path's [M, N] sums, or the packed decode path's
    // per-split sums (64 < M <= 128); the region serves whichever the call takes
    const bool may_split = M > 64 && ((M + 127) / 128) * ((N + 127) / 128) < 256;
    size_t part = may_split ? sizeof(int32_t) * (size_t)(M * N) : 0;
    part = std::max(part, decode_partial_bytes(M, N, K));
    w.counters = w.partial + align256(part);
    const size_t tiles = (size_t)(((M + 127) / 128) * ((N + 127) / 128));
    w.total = w.counters + (may_split ? align256(sizeof(uint32_t) * tiles) : 0);
    return w;
}

}  // namespace lq

using namespace lq;

extern "C" {

int lq_row_sums_i8(const int8_t* d_X, int64_t ld, int64_t rows, int64_t K, int32_t* d_sums,
                   void* stream) {
    LQ_REQUIRE(rows >= 0 && K >= 0 && ld >= K, "lq_row_sums_i8: bad shape");
    if (rows == 0) return LQ_OK;
    LQ_REQUIRE(d_sums && (K == 0 || d_X), "lq_row_sums_i8: NULL pointer");
    hipLaunchKernelGGL(row_sums_i8_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                       as_stream(stream), d_X, ld, rows, K, d_sums);
    return launch_status("lq_row_sums_i8");
}

size_t lq_packed_weights_size(int64_t N, int64_t K) {
    if (N < 0 || K < 0) return 0;
    return (size_t)((N + 15) / 16) * (size_t)((K + 63) / 64) * PACK_TILE;
}

int lq_pack_weights_i8(const int8_t* d_B, int64_t ldb, int64_t N, int64_t K, int8_t* d_packed,
                       void* stream) {
    LQ_REQUIRE(N >= 0 && K >= 0 && ldb >= K, "lq_pack_weights_i8: bad shape");
    LQ_REQUIRE(N <= 0x7fffffff && K <= 0x7fffffff, "lq_pack_weights_i8: size too large");
    const int64_t chunks = (int64_t)lq_packed_weights_size(N, K) / 16;
    if (chunks == 0) return LQ_OK;
    LQ_REQUIRE(d_B && d_packed, "lq_pack_weights_i8: NULL pointer");
    LQ_REQUIRE(aligned16(d_packed), "lq_pack_weights_i8: packed buffer must be 16-byte aligned");
    hipLaunchKernelGGL(pack_weights_i8_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0,
                       as_stream(stream), d_B, ldb, (int)N, (int)K, (int)((K + 63) / 64), chunks,
                       d_packed);
    return launch_status("lq_pack_weights_i8");
}

size_t lq_gemm_w8a8_workspace_size(int64_t M, int64_t N, int64_t K) {
    if (M < 0 || N < 0 || K < 0) return 0;
    return gemm_ws(M, N, K).total;
}

}  // extern "C"

namespace lq {

// Shared validation / setup of lq_gemm_w8a8 and lq_gemm_w8a8_packed.
static int gemm_entry(bool packed, const int8_t* d_A, int64_t lda, const int8_t* d_B, int64_t ldb,
                      void* d_C, int64_t ldc, int64_t M, int64_t N, int64_t K, const float* d_a_scale,
                      int64_t a_scale_stride, const float* d_b_scale, int64_t b_scale_stride,
                      const float* d_a_zero_point, const float* d_b_zero_point, const int32_t* d_b_sums,
                      const float* d_bias, const float* d_out_scale, const float* d_out_zero_point,
                      int out_qmin, int out_qmax, int out_kind, int flags, void* d_workspace,
                      size_t workspace_bytes, void* stream, int2* extrema = nullptr, int* ext_parts = nullptr) {
    LQ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "lq_gemm_w8a8: negative size");
    LQ_REQUIRE(M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff, "lq_gemm_w8a8: size too large");
    if (M == 0 || N == 0) return LQ_OK;
    LQ_REQUIRE(d_C, "lq_gemm_w8a8: NULL output");
    LQ_REQUIRE(K == 0 || (d_A && d_B), "lq_gemm_w8a8: NULL operand");
    LQ_REQUIRE(lda >= K && ldc >= N && (packed || ldb >= K), "lq_gemm_w8a8: leading dimension too small");
    LQ_REQUIRE(valid_out_kind(out_kind), "lq_gemm_w8a8: bad out_kind");
    LQ_REQUIRE(a_scale_stride == 0 || a_scale_stride == 1, "lq_gemm_w8a8: a_scale_stride must be 0 or 1");
    LQ_REQUIRE(b_scale_stride == 0 || b_scale_stride == 1, "lq_gemm_w8a8: b_scale_stride must be 0 or 1");
    const bool requant = out_kind == LQ_OUT_Q8 || out_kind == LQ_OUT_QU8 || out_kind == LQ_OUT_Q16 ||
                         out_kind == LQ_OUT_QU8S8 || out_kind == LQ_OUT_FQ32;
    LQ_REQUIRE(!requant || d_out_scale, "lq_gemm_w8a8: requantizing output needs d_out_scale");
    LQ_REQUIRE(!requant || out_qmax >= out_qmin, "lq_gemm_w8a8: out_qmax < out_qmin");
    LQ_REQUIRE((flags & ~(LQ_EPI_RELU | LQ_EPI_A_U8S8 | LQ_EPI_GELU)) == 0, "lq_gemm_w8a8: unknown flags");
    LQ_REQUIRE(!(flags & LQ_EPI_GELU) || (out_kind == LQ_OUT_F32 && !(flags & LQ_EPI_RELU)),
               "lq_gemm_w8a8: LQ_EPI_GELU needs float32 output and no ReLU");
    const bool has_za = d_a_zero_point != nullptr || (flags & LQ_EPI_A_U8S8);
    if (packed) {
        if (M > 128) return set_error(LQ_ERR_UNSUPPORTED, "lq_gemm_w8a8_packed: M > 128 (use lq_gemm_w8a8)");
        LQ_REQUIRE(K % 16 == 0 && lda % 16 == 0 && aligned16(d_A) && aligned16(d_B),
                   "lq_gemm_w8a8_packed: needs K and lda multiples of 16 and 16-byte aligned A / packed B");
        LQ_REQUIRE(!has_za || d_b_sums,
                   "lq_gemm_w8a8_packed: an activation zero point needs the cached weight sums d_b_sums");
    }
    const GemmWs ws = gemm_ws(M, N, K);
    LQ_REQUIRE(d_workspace || workspace_bytes == 0, "lq_gemm_w8a8: NULL workspace with nonzero size");
    const bool need_asums = d_b_zero_point != nullptr;
    const bool need_bsums = has_za && d_b_sums == nullptr;
    if (need_asums || need_bsums)
        LQ_REQUIRE(d_workspace && workspace_bytes >= ws.partial,
                   "lq_gemm_w8a8: zero-point correction needs the workspace (lq_gemm_w8a8_workspace_size)");

    hipStream_t st = as_stream(stream);
    GemmArgs a{};
    a.A = d_A;
    a.B = d_B;
    a.C = d_C;
    a.lda = lda;
    a.ldb = packed ? K : ldb;
    a.ldc = ldc;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.a_scale = d_a_scale;
    a.b_scale = d_b_scale;
    a.a_stride = (int)a_scale_stride;
    a.b_stride = (int)b_scale_stride;
    a.a_zp = d_a_zero_point;
    a.b_zp = d_b_zero_point;
    a.bias = d_bias;
    a.out_scale = d_out_scale;
    a.out_zp = d_out_zero_point;
    a.qmin = out_qmin;
    a.qmax = out_qmax;
    a.out_kind = out_kind;
    a.relu = (flags & LQ_EPI_RELU) ? 1 : 0;
    a.gelu = (flags & LQ_EPI_GELU) ? 1 : 0;
    a.a_u8s8 = (flags & LQ_EPI_A_U8S8) ? 1 : 0;
    a.splits = 1;
    a.extrema = extrema;
    if (extrema && (packed || out_kind != LQ_OUT_F32)) return GEMM_NO_EXTREMA;
    char* wsb = (char*)d_workspace;
    int rc;
    if (need_asums) {
        a.a_sums = (int32_t*)(wsb + ws.a_sums);
        if ((rc = lq_row_sums_i8(d_A, lda, M, K, (int32_t*)a.a_sums, stream))) return rc;
    }
    if (has_za) {
        if (d_b_sums) {
            a.b_sums = d_b_sums;
        } else {
            a.b_sums = (int32_t*)(wsb + ws.b_sums);
            if ((rc = lq_row_sums_i8(d_B, ldb, N, K, (int32_t*)a.b_sums, stream))) return rc;
        }
    }
    if (packed) {
        if (M >= DEC_MIN_M && d_workspace && workspace_bytes >= ws.counters &&
            ws.counters - ws.partial >= decode_partial_bytes(M, N, K) && (int64_t)M * lda < ((int64_t)1 << 31))
            a.partial = (int32_t*)(wsb + ws.partial);
        switch (out_kind) {
        case LQ_OUT_I32: return launch_packed_skinny<LQ_OUT_I32>(a, st);
        case LQ_OUT_F32: return launch_packed_skinny<LQ_OUT_F32>(a, st);
        case LQ_OUT_F16: return launch_packed_skinny<LQ_OUT_F16>(a, st);
        case LQ_OUT_Q8: return launch_packed_skinny<LQ_OUT_Q8>(a, st);
        case LQ_OUT_QU8: return launch_packed_skinny<LQ_OUT_QU8>(a, st);
        case LQ_OUT_FQ32: return launch_packed_skinny<LQ_OUT_FQ32>(a, st);
        case LQ_OUT_Q16: return launch_packed_skinny<LQ_OUT_Q16>(a, st);
        case LQ_OUT_QU8S8: return launch_packed_skinny<LQ_OUT_QU8S8>(a, st);
        default: return set_error(LQ_ERR_INVALID, "lq_gemm_w8a8: bad out_kind");
        }
    }
    int64_t split_bytes = 0;
    if (d_workspace && workspace_bytes >= ws.total && ws.total > ws.counters) {
        a.partial = (int32_t*)(wsb + ws.partial);
        a.counters = (uint32_t*)(wsb + ws.counters);
        split_bytes = (int64_t)(ws.total - ws.partial);
    }
    switch (out_kind) {
    case LQ_OUT_I32: return GemmLaunch<LQ_OUT_I32>::run(a, st, split_bytes);
    case LQ_OUT_F32: return GemmLaunch<LQ_OUT_F32>::run(a, st, split_bytes, ext_parts);
    case LQ_OUT_F16: return GemmLaunch<LQ_OUT_F16>::run(a, st, split_bytes);
    case LQ_OUT_Q8: return GemmLaunch<LQ_OUT_Q8>::run(a, st, split_bytes);
    case LQ_OUT_QU8: return GemmLaunch<LQ_OUT_QU8>::run(a, st, split_bytes);
    case LQ_OUT_FQ32: return GemmLaunch<LQ_OUT_FQ32>::run(a, st, split_bytes);
    case LQ_OUT_Q16: return GemmLaunch<LQ_OUT_Q16>::run(a, st, split_bytes);
    case LQ_OUT_QU8S8: return GemmLaunch<LQ_OUT_QU8S8>::run(a, st, split_bytes);
    default: return set_error(LQ_ERR_INVALID, "lq_gemm_w8a8: bad out_kind");
    }
}

}  // namespace lq

extern "C" {

int lq_gemm_w8a8(const int8_t* d_A, int64_t lda, const int8_t* d_B, int64_t ldb, void* d_C,
                 int64_t ldc, int64_t M, int64_t N, int64_t K, const float* d_a_scale,
                 int64_t a_scale_stride, const float* d_b_scale, int64_t b_scale_stride,
                 const float* d_a_zero_point, const float* d_b_zero_point, const int32_t* d_b_sums,
                 const float* d_bias, const float* d_out_scale, const float* d_out_zero_point,
                 int out_qmin, int out_qmax, int out_kind, int flags, void* d_workspace,
                 size_t workspace_bytes, void* stream) {
    return gemm_entry(false, d_A, lda, d_B, ldb, d_C, ldc, M, N, K, d_a_scale, a_scale_stride, d_b_scale,
                      b_scale_stride, d_a_zero_point, d_b_zero_point, d_b_sums, d_bias, d_out_scale,
                      d_out_zero_point, out_qmin, out_qmax, out_kind, flags, d_workspace, workspace_bytes,
                      stream);
}

size_t lq_gemm_w8a8_dynamic_quantize_workspace_size(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K < 0) return 0;
    const size_t g = (lq_gemm_w8a8_workspace_size(M, N, K) + 255) & ~(size_t)255;
    const size_t parts = sizeof(int2) * DYN_PARTS_MAX, dq = lq_dynamic_quantize_workspace_size(M * N);
    return g + (parts > dq ? parts : dq);
}

int lq_gemm_w8a8_dynamic_quantize(const int8_t* d_A, int64_t lda, const int8_t* d_B, int64_t ldb, float* d_y,
                                  int64_t M, int64_t N, int64_t K, const float* d_a_scale, int64_t a_scale_stride,
                                  const float* d_b_scale, int64_t b_scale_stride, const float* d_a_zero_point,
                                  const float* d_b_zero_point, const int32_t* d_b_sums, const float* d_bias, int flags,
                                  int q_dtype, int qmin, int qmax, float eps, float* d_qparams, void* d_codes,
                                  void* d_workspace, size_t workspace_bytes, void* stream) {
    const char* fn = "lq_gemm_w8a8_dynamic_quantize";
    LQ_REQUIRE(M > 0 && N > 0 && d_y && d_qparams && d_codes && qmax > qmin, std::string(fn) + ": bad arguments");
    LQ_REQUIRE(d_workspace && workspace_bytes >= lq_gemm_w8a8_dynamic_quantize_workspace_size(M, N, K),
               std::string(fn) + ": workspace too small");
    const size_t g = (lq_gemm_w8a8_workspace_size(M, N, K) + 255) & ~(size_t)255;
    void* tail = static_cast<char*>(d_workspace) + g;
    const size_t tail_bytes = workspace_bytes - g;
    int2* parts = static_cast<int2*>(tail);
    if (dyn_parts_ok(q_dtype, d_y, d_codes, M * N, 1)) {
        int nparts = 0;
        const int rc = gemm_entry(false, d_A, lda, d_B, ldb, d_y, N, M, N, K, d_a_scale, a_scale_stride, d_b_scale,
                                  b_scale_stride, d_a_zero_point, d_b_zero_point, d_b_sums, d_bias, nullptr, nullptr,
                                  0, 0, LQ_OUT_F32, flags, d_workspace, g, stream, parts, &nparts);
        if (rc == LQ_OK && nparts >= 1) {
            const int rq = dyn_quantize_parts(d_y, M * N, q_dtype, qmin, qmax, eps, parts, nparts, d_qparams, d_codes,
                                              as_stream(stream));
            if (rq) return rq;
            note_path("gemm dma with extrema + dynamic quantize");
            return LQ_OK;
        }
        if (rc != GEMM_NO_EXTREMA) return rc;
    }
    // the separate calls
    int rc = gemm_entry(false, d_A, lda, d_B, ldb, d_y, N, M, N, K, d_a_scale, a_scale_stride, d_b_scale,
                        b_scale_stride, d_a_zero_point, d_b_zero_point, d_b_sums, d_bias, nullptr, nullptr, 0, 0,
                        LQ_OUT_F32, flags, d_workspace, g, stream);
    if (rc) return rc;
    return lq_dynamic_quantize_f32(d_y, M * N, q_dtype, qmin, qmax, eps, d_qparams, d_codes, tail, tail_bytes, stream);
}

int lq_gemm_w8a8_packed(const int8_t* d_A, int64_t lda, const int8_t* d_B_packed, void* d_C, int64_t ldc,
                        int64_t M, int64_t N, int64_t K, const float* d_a_scale, int64_t a_scale_stride,
                        const float* d_b_scale, int64_t b_scale_stride, const float* d_a_zero_point,
                        const float* d_b_zero_point, const int32_t* d_b_sums, const float* d_bias,
                        const float* d_out_scale, const float* d_out_zero_point, int out_qmin,
                        int out_qmax, int out_kind, int flags, void* d_workspace, size_t workspace_bytes,
                        void* stream) {
    return gemm_entry(true, d_A, lda, d_B_packed, K, d_C, ldc, M, N, K, d_a_scale, a_scale_stride,
                      d_b_scale, b_scale_stride, d_a_zero_point, d_b_zero_point, d_b_sums, d_bias,
                      d_out_scale, d_out_zero_point, out_qmin, out_qmax, out_kind, flags, d_workspace,
                      workspace_bytes, stream);
}

int lq_dynamic_linear_packed_f32(const float* d_x, int64_t ldx, const float* d_res, int64_t ldres, float* d_sum,
                                 int64_t ld_sum, int src, const float* d_gamma, const float* d_beta, float ln_eps,
                                 int64_t M, int64_t K, int qmin, int qmax, float eps, float* d_qparams,
                                 const int8_t* d_w_packed, const float* d_w_scale, const int32_t* d_w_sums,
                                 const float* d_bias, int64_t N, float* d_y, int64_t ldy, int flags, void* stream) {
    const char* fn = "lq_dynamic_linear_packed_f32";
    LQ_REQUIRE(src == DL_PLAIN || src == DL_LN || src == DL_ADD_LN, std::string(fn) + ": bad src");
    LQ_REQUIRE(M >= 1 && N >= 1 && K >= 16 && ldx >= K && ldy >= N, std::string(fn) + ": bad shape");
    LQ_REQUIRE(d_x && d_w_packed && d_w_scale && d_w_sums && d_y, std::string(fn) + ": NULL pointer");
    LQ_REQUIRE(src != DL_ADD_LN || (d_res && ldres >= K), std::string(fn) + ": DL_ADD_LN needs res");
    LQ_REQUIRE(!d_sum || (src == DL_ADD_LN && ld_sum >= K), std::string(fn) + ": sum only with DL_ADD_LN");
    LQ_REQUIRE(0 <= qmin && qmin < qmax && qmax <= 255, std::string(fn) + ": an unsigned 8-bit grid expected");
    LQ_REQUIRE((flags & ~LQ_EPI_GELU) == 0, std::string(fn) + ": flags other than LQ_EPI_GELU");
    if (M > 16 || K % 16 != 0 || M * K > DL_MAX_MK || (src != DL_PLAIN && (K > DL_MAX_K_LN || M * K > DL_MAX_MK_LN)))
        return set_error(LQ_ERR_UNSUPPORTED, std::string(fn) + ": outside the one-launch sizes (M <= 16, K % 16 == 0, "
                                                           "M K <= 16384, with a norm K <= 2048 and M K <= 8192)");
    if (src == DL_PLAIN && (ldx % 4 != 0 || (reinterpret_cast<uintptr_t>(d_x) & 15) != 0))
        return set_error(LQ_ERR_UNSUPPORTED, std::string(fn) + ": x rows must be 16-byte aligned");
    GemmArgs a{};
    a.B = d_w_packed;
    a.C = d_y;
    a.ldc = ldy;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.b_scale = d_w_scale;
    a.b_stride = 1;
    a.b_sums = d_w_sums;
    a.bias = d_bias;
    a.out_kind = LQ_OUT_F32;
    a.gelu = (flags & LQ_EPI_GELU) != 0;
    a.a_u8s8 = 1;
    a.splits = 1;
    DynLinArgs dl;
    dl.x = d_x;
    dl.ldx = ldx;
    dl.res = d_res;
    dl.ldres = ldres;
    dl.sum = d_sum;
    dl.ldsum = ld_sum;
    dl.gamma = d_gamma;
    dl.beta = d_beta;
    dl.ln_eps = ln_eps;
    dl.qmin = qmin;
    dl.eps = eps;
    dl.width_f = (float)(qmax - qmin);
    dl.g = make_grid(qmin, qmax);
    dl.qp = d_qparams;
    const int KS = (int)((K + 63) / 64);
    dl.KP = KS * 64 + 16;
    const size_t lds = (size_t)((M * dl.KP + 15) & ~15) + (src == DL_PLAIN ? 0 : (size_t)4 * M * K);
    const int64_t tiles = (N + 15) / 16;
    const bool wt = tiles >= DL_WT_MIN_TILES;
    const dim3 grid((unsigned)(wt ? (tiles + 3) / 4 : tiles)), block(256);
    const hipStream_t st = as_stream(stream);
    auto go = [&](auto src_c, auto wt_c, auto maxc_c, auto rpw_c) {
        constexpr int S = decltype(src_c)::value, C = decltype(maxc_c)::value, R = decltype(rpw_c)::value;
        constexpr bool W = decltype(wt_c)::value;
        hipLaunchKernelGGL((dyn_linear_skinny_kernel<S, W, C, R, LQ_OUT_F32>), grid, block, lds, st, dl, a);
    };
    auto by_src = [&](auto wt_c) {
        using I = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        using I4 = std::integral_constant<int, 4>;
        using I8 = std::integral_constant<int, 8>;
        // (chunks per lane, rows per wave): M <= 16, and M K <= 8192 keeps M <= 7 past K = 1024
        auto normed = [&](auto src_c) {
            if (K <= 2 * 4 * LN_T) go(src_c, wt_c, I2{}, I4{});
            else if (K <= 4 * 4 * LN_T) go(src_c, wt_c, I4{}, I4{});
            else go(src_c, wt_c, I8{}, I2{});
        };
        if (src == DL_PLAIN) go(std::integral_constant<int, DL_PLAIN>{}, wt_c, I{}, I{});
        else if (src == DL_LN) normed(std::integral_constant<int, DL_LN>{});
        else normed(std::integral_constant<int, DL_ADD_LN>{});
    };
    if (wt) by_src(std::true_type{});
    else by_src(std::false_type{});
    note_path(wt ? "dynamic linear one launch, wave tiles" : "dynamic linear one launch, split k");
    return launch_status(fn);
}

}  // extern "C"

// ------------------------------------------------------ allocation-free variant
//
// lq_gemm_w8a8_noalloc keeps the workspace of lq_gemm_w8a8 (the activation / weight code
// sums, split-K partial sums and tile arrival counters) in this file-scope device array
// instead of a caller buffer, for callers that cannot allocate (graph capture, serving
// loops).  Each GPU the library runs on holds its own copy until the process ends; every
// call on one GPU shares it, so calls that overlap on one GPU race.  Nothing in it is
// assumed to persist: the code sums are recomputed and the split-K partials and counters are
// cleared by a fill kernel inside each call that uses them.
constexpr size_t LQ_NOALLOC_SCRATCH_BYTES = (size_t)16 << 20;
static __device__ __align__(256) uint8_t scratch[LQ_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[NOALLOC_MAX_DEVICES];  // device address of `scratch` on each device

// The device address of this GPU's `scratch`, looked up once per device with that device
// current (the array's host-side name is not a device address).
int current_device_scratch(void** out) {
    int dev = 0;
    LQ_HIP(hipGetDevice(&dev));
    LQ_REQUIRE(dev >= 0 && dev < NOALLOC_MAX_DEVICES, "lq_gemm_w8a8_noalloc: device index out of range");
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return check_hip(e, "lq_gemm_w8a8_noalloc: hipGetSymbolAddress(scratch)");
        if (!p) return set_error(LQ_ERR_HIP, "lq_gemm_w8a8_noalloc: no device address for scratch");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return LQ_OK;
}
}  // namespace

extern "C" {

size_t lq_gemm_w8a8_noalloc_scratch_bytes(void) { return LQ_NOALLOC_SCRATCH_BYTES; }

int lq_gemm_w8a8_noalloc(const int8_t* d_A, int64_t lda, const int8_t* d_B, int64_t ldb, void* d_C,
                         int64_t ldc, int64_t M, int64_t N, int64_t K, const float* d_a_scale,
                         int64_t a_scale_stride, const float* d_b_scale, int64_t b_scale_stride,
                         const float* d_a_zero_point, const float* d_b_zero_point,
                         const int32_t* d_b_sums, const float* d_bias, const float* d_out_scale,
                         const float* d_out_zero_point, int out_qmin, int out_qmax, int out_kind,
                         int flags, void* stream) {
    const size_t need = lq_gemm_w8a8_workspace_size(M, N, K);
    if (need > LQ_NOALLOC_SCRATCH_BYTES)
        return set_error(LQ_ERR_UNSUPPORTED,
                         "lq_gemm_w8a8_noalloc: this shape needs " + std::to_string(need) +
                             " bytes of scratch, more than the " + std::to_string(LQ_NOALLOC_SCRATCH_BYTES) +
                             " the library holds per GPU (use lq_gemm_w8a8 with a workspace)");
    void* ws = nullptr;
    if (const int rc = current_device_scratch(&ws)) return rc;
    return gemm_entry(false, d_A, lda, d_B, ldb, d_C, ldc, M, N, K, d_a_scale, a_scale_stride, d_b_scale,
                      b_scale_stride, d_a_zero_point, d_b_zero_point, d_b_sums, d_bias, d_out_scale,
                      d_out_zero_point, out_qmin, out_qmax, out_kind, flags, ws, LQ_NOALLOC_SCRATCH_BYTES,
                      stream);
}

}  // extern "C"
