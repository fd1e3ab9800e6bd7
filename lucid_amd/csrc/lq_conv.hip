// lq_conv.hip -- int8 Conv2d as an implicit GEMM on CDNA4 MFMA (v_mfma_i32_16x16x64_i8), with
// the W8A8 epilogue of the GEMM, plus the float direct convolution and eval BatchNorm the
// float model runs during calibration.
//
// Replaces the compute of Lucid's quantized Conv2d, which dequantizes the int8 kernel and runs
// a float conv (im2col + sgemm per batch and group) every call, then fake-quantizes
// (lucid/nn/quantized/conv.py:137-172 -> lucid/nn/functional/conv.py:53-84 ->
// lucid/_C/backend/cpu/methods/Conv.cpp:271-360).  Here:
//
//   acc[p, co] = sum_{kh,kw,c} (x[n, c, oh*sh + kh*dh - pt, ow*sw + kw*dw - pl] - za) * w[co, c, kh, kw]
//
// exact in int32, then y = fl32(fl32(float(acc) * fl32(sx * sw[co])) + b[co]), ReLU, requantize.
//
// Data layout.  The activation codes (NCHW, as the module API holds them) are first packed
// into a padded NHWC copy, x_p[n][hp][wp][g][cp] with cp padded to a multiple of 16: the
// spatial border (zeros padding) and the channel padding hold the activation zero point in
// its stored units, so they contribute exactly 0 to acc; reflect / replicate / circular
// padding are index maps of the same pack.  The weights are packed once per module into
// w_p[g][co][kh][kw][cp] (zero channel padding) with their code sums (the zero-point term).
// A 16-byte K chunk of the implicit im2col row of pixel p is then one contiguous load:
// K index k = (kh * KW + kw) * Cp + c, chunk start c a multiple of 16.
//
// Tiling.  A workgroup (4 waves) computes 128 pixels x 64 output channels of one group with
// K steps of 64 bytes, register-staged double buffering through LDS (16-byte chunks XOR-
// swizzled by row so the MFMA fragment reads are conflict-free).  Pixels are the MFMA row
// operand, so a lane's four results are four consecutive pixels of one output channel:
// one contiguous NCHW store.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <utility>

#include "lq_dma.h"
#include "lq_epilogue.h"
#include "lq_internal.h"

namespace lq {
namespace {

constexpr int CV_BM = 128, CV_BN = 64, CV_BK = 64, CV_THREADS = 256;

// ---------------------------------------------------------------- packing

__device__ __forceinline__ int pad_index(int i, int n, int mode) {
    // source index of padded coordinate i (may be < 0 or >= n), or -1 for a zero-padded tap
    if (i >= 0 && i < n) return i;
    switch (mode) {
        case LQ_PAD_REFLECT: {  // mirror without repeating the edge
            if (n == 1) return 0;
            const int period = 2 * (n - 1);
            int j = i % period;
            if (j < 0) j += period;
            return j < n ? j : period - j;
        }
        case LQ_PAD_REPLICATE: return i < 0 ? 0 : n - 1;
        case LQ_PAD_CIRCULAR: {
            int j = i % n;
            return j < 0 ? j + n : j;
        }
        default: return -1;
    }
}

struct PackArgs {
    const int8_t* x;
    int8_t* xp;
    int N, C, H, W, G, Cg, Cp, Hp, Wp, pt, pl, mode;
    const float* a_zp;
    int a_u8s8;
};

// The padded NHWC copy in one launch.  Workgroups [0, tiles) fill the interior as a
// transpose through LDS: a workgroup takes 256 consecutive positions p of one image plane
// (the flattened h * W + w, so rows of any width fill the tile) and CV_PCB channels; a lane
// loads the same dword (4 positions) of 4 consecutive channels, transposes the 4 x 4 bytes in
// registers (v_perm) and stores 4 channel dwords to LDS; the workgroup then writes 16-byte
// channel chunks at the padded position of each p.  Channels past Cg take the fill code (the
// zero point).  The remaining workgroups gather the border positions (rows above / below the
// image, columns left / right of it) -- or, for planes under half a tile, every padded
// position: the fill code for zeros padding, else the (reflect / replicate / circular)
// source, one thread per 16 channels of a position.
constexpr int CV_PCB = 64;             // channels per interior workgroup
constexpr int CV_PROW = CV_PCB + 4;    // LDS bytes per position (odd word stride)

struct PackGeom {
    int tiles;          // interior workgroups per (n, g): positions x channel tiles
    int ptiles;         // position tiles per plane
    int pb, pr;         // bottom / right padding
    int border_cells;   // gathered positions per (n, g) image
    int all_cells;      // gather every padded position (small planes), no interior tiles
};

template <bool DWORD>
__global__ __launch_bounds__(256) void conv_pack_input_kernel(PackArgs a, PackGeom pg) {
    const int nb = blockIdx.y;
    const int n = nb / a.G, g = nb - n * a.G;
    const int fill = (a.a_zp ? (int)a.a_zp[0] : 0) - (a.a_u8s8 ? 128 : 0);
    const int8_t* plane0 = a.x + ((int64_t)n * a.C + (int64_t)g * a.Cg) * a.H * a.W;
    if ((int)blockIdx.x >= pg.tiles) {
        // border positions of image (n, g)
        const int chunks = a.Cp / 16;
        const int id = ((int)blockIdx.x - pg.tiles) * 256 + threadIdx.x;
        if (id >= pg.border_cells * chunks) return;
        const int j = id % chunks, cell = id / chunks;
        const int rowcells = (a.pt + pg.pb) * a.Wp;
        int hp, wp;
        if (pg.all_cells) {
            hp = cell / a.Wp;
            wp = cell - hp * a.Wp;
        } else if (cell < rowcells) {
            const int br = cell / a.Wp;
            hp = br < a.pt ? br : a.pt + a.H + (br - a.pt);
            wp = cell - br * a.Wp;
        } else {
            const int c2 = cell - rowcells, side = a.pl + pg.pr;
            const int row = c2 / side, k = c2 - row * side;
            hp = a.pt + row;
            wp = k < a.pl ? k : a.pl + a.W + (k - a.pl);
        }
        const int h = pad_index(hp - a.pt, a.H, a.mode);
        const int w = pad_index(wp - a.pl, a.W, a.mode);
        uint32_t word[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t v = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int c = 16 * j + 4 * q + b;
                int code = fill;
                if (c < a.Cg && h >= 0 && w >= 0) code = plane0[((int64_t)c * a.H + h) * a.W + w];
                v |= (uint32_t)(uint8_t)code << (8 * b);
            }
            word[q] = v;
        }
        const int64_t dst = ((((int64_t)n * a.Hp + hp) * a.Wp + wp) * a.G + g) * a.Cp + 16 * j;
        *reinterpret_cast<vu4*>(a.xp + dst) = vu4{word[0], word[1], word[2], word[3]};
        return;
    }
    __shared__ uint32_t sm[256 * CV_PROW / 4];
    const int HW = a.H * a.W;
    const int ct = (int)blockIdx.x / pg.ptiles;
    const int p0 = ((int)blockIdx.x - ct * pg.ptiles) * 256;
    const int c0 = ct * CV_PCB;
    const int cb = min(CV_PCB, a.Cp - c0);  // a multiple of 16
    const uint32_t fill4 = (uint32_t)(uint8_t)fill * 0x01010101u;
    const int d = threadIdx.x & 63;  // dword of the tile row: positions p .. p + 3
    const int p = p0 + 4 * d;
    constexpr int GROUPS = CV_PCB / 16;  // 4-channel groups per lane, all loads issued first
    uint32_t v[GROUPS][4];
#pragma unroll
    for (int k = 0; k < GROUPS; ++k) {
        const int rg = (threadIdx.x >> 6) + 4 * k;  // channels 4 rg .. 4 rg + 3 of the tile
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int c = c0 + 4 * rg + e;
            uint32_t t = fill4;
            if (4 * rg < cb && c < a.Cg) {
                const int8_t* src = plane0 + (int64_t)c * HW + p;
                if (DWORD) {
                    if (p < HW) t = *reinterpret_cast<const uint32_t*>(src);
                } else {
                    t = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) t |= (uint32_t)(uint8_t)(p + i < HW ? src[i] : (int8_t)0) << (8 * i);
                }
            }
            v[k][e] = t;
        }
    }
#pragma unroll
    for (int k = 0; k < GROUPS; ++k) {
        const int rg = (threadIdx.x >> 6) + 4 * k;
        if (4 * rg >= cb) continue;
        // 4 x 4 byte transpose: row e = channel, byte i = position -> dword i = position
        const uint32_t ab_lo = __builtin_amdgcn_perm(v[k][1], v[k][0], 0x05010400u);
        const uint32_t ab_hi = __builtin_amdgcn_perm(v[k][1], v[k][0], 0x07030602u);
        const uint32_t cd_lo = __builtin_amdgcn_perm(v[k][3], v[k][2], 0x05010400u);
        const uint32_t cd_hi = __builtin_amdgcn_perm(v[k][3], v[k][2], 0x07030602u);
        const uint32_t o[4] = {__builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u),
                               __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u),
                               __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u),
                               __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u)};
#pragma unroll
        for (int i = 0; i < 4; ++i) sm[((4 * d + i) * CV_PROW) / 4 + rg] = o[i];
    }
    __syncthreads();
    const int chunks = cb / 16;
    const int64_t GCp = (int64_t)a.G * a.Cp;
    for (int j = threadIdx.x; j < 256 * chunks; j += 256) {
        const int pl = j / chunks, cc = j - pl * chunks;
        const int pp = p0 + pl;
        if (pp >= HW) continue;
        const int h = pp / a.W, w = pp - h * a.W;
        const uint32_t* q = sm + (pl * CV_PROW) / 4 + 4 * cc;
        const int64_t dst = (((int64_t)n * a.Hp + h + a.pt) * a.Wp + w + a.pl) * GCp + (int64_t)g * a.Cp + c0 + cc * 16;
        *reinterpret_cast<vu4*>(a.xp + dst) = vu4{q[0], q[1], q[2], q[3]};
    }
}

// ---------------------------------------------------------------- tap-im2col form
//
// Inputs with 2..4 channels per group (images) waste most of a 16-channel padded position.
// For them the KW taps of a kernel row and the channels are packed together: position
// (n, hp, ow) of the packed input holds, per group, the 32 bytes
//   xt[j = kw * Cg + c] = x[n][g Cg + c][hp - pt][ow sw + kw dw - pl]   (j < KW Cg; the rest fill)
// and the convolution runs as a KH x 1 one over 32 channels at horizontal stride 1:
// K = KH x 32 (the ResNet stem, 7x7 over 3 channels: 224 bytes = 2 stages instead of
// 7 x 7 x 16 = 784 = 7).  Weight rows are [co][kh * 32 + kw * Cg + c].  The form depends only on
// what the weight pack knows (channels per group and KW), so the pack and the call agree;
// one channel per group (depthwise) keeps the plain form.
__host__ __device__ constexpr bool conv_taps_form(int64_t Cg, int64_t KW) {
    return Cg >= 2 && Cg <= 4 && KW >= 2 && Cg * KW <= 32;
}
constexpr int CV_TAPS_CP = 32;        // bytes per position and group in the tap-im2col form
constexpr int CV_TAPS_OWB = 128;      // output columns per pack workgroup (two chunks each)
constexpr int CV_TAPS_SPAN = 512;     // input bytes of one channel row staged per workgroup

struct TapsArgs {
    const int8_t* x;
    int8_t* xp;
    int N, C, H, W, G, Cg, Hp, OW, KW, sw, dw, pt, pl, mode;
    int owb, span;  // output columns per workgroup, staged input bytes per channel
    const float* a_zp;
    int a_u8s8;
};

// One workgroup per (image n, CV_TAPS_ROWS consecutive padded rows, column block): per group,
// the Cg input rows each padded row reads are staged in LDS (padding sources resolved), then
// each thread writes 16-byte halves of 32-byte positions.  A thread always writes the same
// half (the item stride is even), so its 16 byte offsets into a staged row are computed once.
constexpr int CV_TAPS_ROWS = 4;

__global__ __launch_bounds__(256) void conv_pack_taps_kernel(TapsArgs a) {
    __shared__ int8_t rows[CV_TAPS_ROWS * 4 * CV_TAPS_SPAN];  // rows x Cg (<= 4) x span
    const int hblocks = (a.Hp + CV_TAPS_ROWS - 1) / CV_TAPS_ROWS;
    const int n = blockIdx.x / hblocks, hp0 = (blockIdx.x - n * hblocks) * CV_TAPS_ROWS;
    const int ow0 = blockIdx.y * a.owb;
    const int fill = (a.a_zp ? (int)a.a_zp[0] : 0) - (a.a_u8s8 ? 128 : 0);
    const int col0 = ow0 * a.sw - a.pl;  // input column of staged byte 0
    const int rowbytes = a.Cg * a.span;  // one padded row's staged channels
    // byte b of this thread's half: staged offset c * span + kw * dw, or -1 (fill)
    const int half = threadIdx.x & 1;
    int off[16];
    {
        int kw = (half * 16) / a.Cg, c = half * 16 - kw * a.Cg;
#pragma unroll
        for (int b = 0; b < 16; ++b) {
            off[b] = kw < a.KW ? c * a.span + kw * a.dw : -1;
            if (++c == a.Cg) {
                c = 0;
                ++kw;
            }
        }
    }
    const int items = CV_TAPS_ROWS * a.owb * 2;
    // staged bytes j = threadIdx.x + 256 jj (span <= 512): their source columns, and the
    // source rows of the block's padded rows, resolved once
    int wsrc[2], hsrc[CV_TAPS_ROWS];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
        const int j = threadIdx.x + 256 * jj;
        wsrc[jj] = j < a.span ? pad_index(col0 + j, a.W, a.mode) : -1;
    }
#pragma unroll
    for (int r = 0; r < CV_TAPS_ROWS; ++r) hsrc[r] = hp0 + r < a.Hp ? pad_index(hp0 + r - a.pt, a.H, a.mode) : -1;
    for (int g = 0; g < a.G; ++g) {
        // every load of the stage first (one memory round trip), then the LDS stores
        int8_t v[CV_TAPS_ROWS][4][2];
#pragma unroll
        for (int r = 0; r < CV_TAPS_ROWS; ++r)
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    v[r][c][jj] = (int8_t)fill;
                    if (c < a.Cg && hsrc[r] >= 0 && wsrc[jj] >= 0)
                        v[r][c][jj] = a.x[(((int64_t)n * a.C + (int64_t)g * a.Cg + c) * a.H + hsrc[r]) * a.W + wsrc[jj]];
                }
#pragma unroll
        for (int r = 0; r < CV_TAPS_ROWS; ++r)
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    const int j = threadIdx.x + 256 * jj;
                    if (c < a.Cg && j < a.span) rows[r * rowbytes + c * a.span + j] = v[r][c][jj];
                }
        __syncthreads();
        for (int it = threadIdx.x; it < items; it += 256) {
            const int pos = it >> 1;
            const int r = pos / a.owb, col = pos - r * a.owb;
            const int hp = hp0 + r, ow = ow0 + col;
            if (hp >= a.Hp || ow >= a.OW) continue;
            const int8_t* row = rows + r * rowbytes + col * a.sw;
            uint32_t word[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t v = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int o = off[4 * q + b];
                    v |= (uint32_t)(uint8_t)(o >= 0 ? (int)row[o] : fill) << (8 * b);
                }
                word[q] = v;
            }
            const int64_t dst = ((((int64_t)n * a.Hp + hp) * a.OW + ow) * a.G + g) * CV_TAPS_CP + half * 16;
            *reinterpret_cast<vu4*>(a.xp + dst) = vu4{word[0], word[1], word[2], word[3]};
        }
        __syncthreads();
    }
}

// Weight rows of the tap-im2col form: one thread per 16-byte chunk of w_p[co][kh * 32 + j].
__global__ __launch_bounds__(256) void conv_pack_weights_taps_kernel(const int8_t* __restrict__ w, int Cout, int Cg,
                                                                     int KH, int KW, int ldw, int8_t* __restrict__ wp) {
    const int chunks = ldw / 16;
    const int64_t total = (int64_t)Cout * chunks;
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= total) return;
    const int64_t co = id / chunks;
    const int k0 = (int)(id - co * chunks) * 16;
    uint32_t word[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t v = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int k = k0 + q * 4 + b;
            const int kh = k / CV_TAPS_CP, j = k - kh * CV_TAPS_CP;
            const int kw = j / Cg, c = j - kw * Cg;
            const int8_t x = (kh < KH && kw < KW) ? w[((co * Cg + c) * KH + kh) * KW + kw] : (int8_t)0;
            v |= (uint32_t)(uint8_t)x << (8 * b);
        }
        word[q] = v;
    }
    reinterpret_cast<vu4*>(wp)[id] = vu4{word[0], word[1], word[2], word[3]};
}

// One thread per 16-byte chunk of a packed weight row w_p[co][k], k = (kh * KW + kw) * Cp + c,
// rows ldw bytes long (K rounded up to whole 128-byte stages, the tail zero).
__global__ __launch_bounds__(256) void conv_pack_weights_kernel(const int8_t* __restrict__ w, int Cout, int Cg,
                                                                int KH, int KW, int Cp, int ldw,
                                                                int8_t* __restrict__ wp) {
    const int chunks = ldw / 16;
    const int64_t total = (int64_t)Cout * chunks;
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= total) return;
    const int64_t co = id / chunks;
    const int k0 = (int)(id - co * chunks) * 16;
    const int tap = k0 / Cp, c0 = k0 - tap * Cp;  // a chunk never crosses a tap (Cp % 16 == 0)
    const int kh = tap / KW, kw = tap - kh * KW;
    uint32_t word[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t v = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int c = c0 + q * 4 + b;
            const int8_t x = (tap < KH * KW && c < Cg) ? w[((co * Cg + c) * KH + kh) * KW + kw] : (int8_t)0;
            v |= (uint32_t)(uint8_t)x << (8 * b);
        }
        word[q] = v;
    }
    reinterpret_cast<vu4*>(wp)[id] = vu4{word[0], word[1], word[2], word[3]};
}

// sums[co] = sum of output channel co's codes (one wave per channel).
__global__ __launch_bounds__(256) void conv_weight_sums_kernel(const int8_t* __restrict__ w, int Cout, int64_t per,
                                                               int32_t* __restrict__ sums) {
    const int co = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (co >= Cout) return;
    const int lane = threadIdx.x & 63;
    int32_t s = 0;
    for (int64_t i = lane; i < per; i += 64) s += w[(int64_t)co * per + i];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) sums[co] = s;
}

// ---------------------------------------------------------------- implicit GEMM

struct ConvArgs {
    const int8_t* xp;
    const int8_t* wp;
    void* y;
    int N, Hp, Wp, G, Cp, Cout_g, KH, KW, sh, sw, dh, dw, OH, OW;
    int K, P, ldw;  // real K; packed weight row stride (K padded to whole 128-byte stages)
    const float* a_scale;
    const float* a_zp;
    int a_u8s8;
    const float* w_scale;
    const int32_t* w_sums;
    const float* bias;
    const float* out_scale;
    const float* out_zp;
    int qmin, qmax, relu;
};

// 16-byte LDS slot of chunk c (0..3) of tile row r: rows are 64 bytes (16 banks); the XOR by
// (r >> 2) & 3 spreads the 16 rows an MFMA fragment read touches over all 64 banks.
__device__ __forceinline__ int cv_slot(int r, int c) { return r * 4 + (c ^ ((r >> 2) & 3)); }

// Running (kh, kw, c) of a K offset, advanced by whole K steps without divisions.
struct KPos {
    int kh, kw, c;
    __device__ __forceinline__ void init(int k, int Cp, int KW) {
        const int khw = k / Cp;
        c = k - khw * Cp;
        kh = khw / KW;
        kw = khw - kh * KW;
    }
    __device__ __forceinline__ void advance(int step, int Cp, int KW) {
        c += step;
        while (c >= Cp) {
            c -= Cp;
            if (++kw == KW) {
                kw = 0;
                ++kh;
            }
        }
    }
};

template <int KIND>
__global__ __launch_bounds__(CV_THREADS) void conv_i8_kernel(ConvArgs a) {
    __shared__ vu4 lds_a[2][CV_BM * 4];
    __shared__ vu4 lds_b[2][CV_BN * 4];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;  // wave: 64 pixels x 32 channels
    const int p0 = blockIdx.x * CV_BM;
    const int co0 = blockIdx.y * CV_BN;
    const int g = blockIdx.z;
    const int GCp = a.G * a.Cp;
    const int T = (a.K + CV_BK - 1) / CV_BK;

    // A: two 16-byte chunks per thread (rows r0, r0 + 64 of the tile, chunk ca)
    const int ca = tid & 3;
    int64_t abase[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int p = min(p0 + (tid >> 2) + 64 * i, a.P - 1);
        const int n = p / (a.OH * a.OW);
        const int rem = p - n * a.OH * a.OW;
        const int oh = rem / a.OW, ow = rem - oh * a.OW;
        abase[i] = (((int64_t)n * a.Hp + (int64_t)oh * a.sh) * a.Wp + (int64_t)ow * a.sw) * GCp + (int64_t)g * a.Cp;
    }
    KPos ka;
    ka.init(16 * ca, a.Cp, a.KW);
    int ka_k = 16 * ca;
    // B: one chunk per thread (row tid >> 2, chunk tid & 3)
    const int brow = tid >> 2;
    const int8_t* bptr = a.wp + ((int64_t)g * a.Cout_g + min(co0 + brow, a.Cout_g - 1)) * a.ldw + 16 * ca;

    vu4 ra[2], rb;
    auto gload = [&](int t) {
        const bool kin = ka_k < a.K;
        const int64_t off = ((int64_t)ka.kh * a.dh * a.Wp + (int64_t)ka.kw * a.dw) * GCp + ka.c;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            ra[i] = kin ? *reinterpret_cast<const vu4*>(a.xp + abase[i] + off) : vu4{0u, 0u, 0u, 0u};
        rb = (t * CV_BK + 16 * ca < a.K) ? *reinterpret_cast<const vu4*>(bptr + (int64_t)t * CV_BK)
                                        : vu4{0u, 0u, 0u, 0u};
        ka.advance(CV_BK, a.Cp, a.KW);
        ka_k += CV_BK;
    };
    auto sstore = [&](int s) {
#pragma unroll
        for (int i = 0; i < 2; ++i) lds_a[s][cv_slot((tid >> 2) + 64 * i, ca)] = ra[i];
        lds_b[s][cv_slot(brow, ca)] = rb;
    };

    v4i acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    gload(0);
    sstore(0);
    __syncthreads();
    const int fr = lane & 15, fc = lane >> 4;  // fragment row / 16-byte chunk
    for (int t = 0; t < T; ++t) {
        const int s = t & 1;
        if (t + 1 < T) gload(t + 1);
        v4i fa[4], fb[2];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const vu4 v = lds_a[s][cv_slot(wm * 64 + i * 16 + fr, fc)];
            fa[i] = __builtin_bit_cast(v4i, v);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const vu4 v = lds_b[s][cv_slot(wn * 32 + j * 16 + fr, fc)];
            fb[j] = __builtin_bit_cast(v4i, v);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        if (t + 1 < T) sstore(s ^ 1);
        __syncthreads();
    }

    // epilogue: lane holds pixels 4*(lane/16) + r of each m-tile, channel lane % 16 of each n-tile
    EpiParams ep;
    ep.za = (a.a_zp ? (int)a.a_zp[0] : 0) - (a.a_u8s8 ? 128 : 0);
    ep.has_za = a.a_zp != nullptr || a.a_u8s8;
    ep.out_s = a.out_scale ? a.out_scale[0] : 1.0f;
    ep.out_inv = 1.0f / ep.out_s;
    ep.out_z = a.out_zp ? a.out_zp[0] : 0.0f;
    ep.g = make_grid(a.qmin, a.qmax);
    const float sa = a.a_scale ? a.a_scale[0] : 1.0f;
    const int OHW = a.OH * a.OW;
    const int Cout = a.G * a.Cout_g;
    constexpr int b = OutTraits<KIND>::bytes;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int col = co0 + wn * 32 + j * 16 + fr;  // channel within the group
        if (col >= a.Cout_g) continue;
        const int co = g * a.Cout_g + col;
        const float sb = a.w_scale[co];
        const float bias = a.bias ? a.bias[co] : 0.0f;
        const int32_t wsum = a.w_sums ? a.w_sums[co] : 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int p = p0 + wm * 64 + i * 16 + 4 * fc;
            if (p >= a.P) continue;
            uint32_t out[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                uint32_t v = (uint32_t)acc[i][j][r];
                if (ep.has_za) v -= (uint32_t)ep.za * (uint32_t)wsum;
                out[r] = epi_one<KIND>((int32_t)v, sa, sb, a.bias ? &bias : nullptr, a.relu != 0, ep);
            }
            const int n = p / OHW, pix = p - n * OHW;
            const int64_t base = ((int64_t)n * Cout + co) * OHW + pix;
            if ((OHW & 3) == 0 && p + 3 < a.P) {  // four pixels of one image, aligned
                if (b == 4) {
                    *reinterpret_cast<vu4*>(reinterpret_cast<uint32_t*>(a.y) + base) = vu4{out[0], out[1], out[2], out[3]};
                } else if (b == 2) {
                    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.y) + base) =
                        make_uint2(out[0] | (out[1] << 16), out[2] | (out[3] << 16));
                } else {
                    *reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(a.y) + base) =
                        out[0] | (out[1] << 8) | (out[2] << 16) | (out[3] << 24);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int pr = p + r;
                    if (pr >= a.P) break;
                    const int nr = pr / OHW, pixr = pr - nr * OHW;
                    store_elem<KIND>(a.y, ((int64_t)nr * Cout + co) * OHW + pixr, out[r]);
                }
            }
        }
    }
}

// ------------------------------------------------- LDS-DMA implicit GEMM (production)
//
// The main loop of the int8 GEMM (lq_gemm.hip) with the im2col rows fetched by LDS-DMA:
// GEMM rows are output pixels, columns output channels of a group, K = (kh, kw, c) over the
// padded NHWC input in whole 128-byte stages (the packed weight rows carry zero columns past
// KH * KW * Cp).  A lane's 16-byte copy of pixel row p, logical chunk k0 + 16 q, comes from
// x_p + base(p) + tap_off(k / Cp) + k % Cp: one contiguous load per lane, any tap, any stride
// or dilation.  Taps past KH * KW (the K padding) read the first tap again; their weights are
// zero.  Pixel fragments are permuted (lane row rho reads tile row (rho / 4) * 16 + 4 j +
// rho % 4), so a lane's results are 16 consecutive pixels of one output channel: one 16-byte
// NCHW store per channel for int8 outputs.
constexpr int CV_MAX_TAPS = 128;
// Stage buffers of the 128 x 64 tile.  Two, like the 256 x 64 tile: a four-stage ring
// (96 KB of LDS, one workgroup per CU) measured 15-30% slower on the ResNet-18 layers than
// two stages with several workgroups per CU.
constexpr int CV_SMALL_NBUF = 2;

struct ConvDmaArgs {
    const int8_t* xp;
    const int8_t* wp;
    void* y;
    uint32_t xp_bytes;
    int Hp, Wp, G, Cp, cp_shift, Cout_g, KH, KW, sh, sw, dh, dw, OH, OW, P, nk, ldw;
    int kw_magic;                  // ceil(2^16 / KW): tap / KW = (tap * kw_magic) >> 16 for tap < 128
    int kh_stride, kw_stride;      // input bytes between vertical / horizontal taps
    const float* a_scale;
    const float* a_zp;
    int a_u8s8;
    const float* w_scale;
    const int32_t* w_sums;
    const float* bias;
    const float* out_scale;
    const float* out_zp;
    int qmin, qmax, relu;
    // split-K: with splits > 1 a first launch (phase 0, gridDim.z = G * splits) leaves each
    // split's exact int32 tile sums in part; a second launch (phase 1, gridDim.z = G) adds
    // them in split order and runs the epilogue
    int splits, phase;
    int32_t* part;
    // NHWC output (lq_conv2d_i8_nhwc): y is pixel (0, 0) of a padded buffer -- ypad border
    // pixels on each side, yrow bytes per padded row, yimg per image, ycs per pixel -- whose
    // border this launch fills with the output grid's zero-point code
    int out_nhwc, ypad, ycs;
    int64_t yrow, yimg;
    // residual merge into the NHWC output (QFunctional.add_relu of the conv's codes and a skip
    // tensor of the same layout): the merge's grid, and the skip's codes and grid
    const int8_t* skip;
    int skip_type, m_type, m_relu;
    const float* skip_scale;
    const float* skip_zp;
    const float* m_scale;
    const float* m_zp;
    int m_qmin, m_qmax;
};

// A stored byte code of an integer output kind / code type as its float code value.
__device__ __forceinline__ float nhwc_code(uint32_t b, int type) {
    if (type == LQ_I8) return (float)(int)(int8_t)(uint8_t)b;
    if (type == LQ_U8) return (float)(int)(uint8_t)b;
    return (float)((int)(int8_t)(uint8_t)b + 128);  // LQ_U8S8: c stored as c - 128
}
__device__ __forceinline__ uint32_t nhwc_store(float t, float inv, float z, const Grid& g, int type) {
    if (type == LQ_I8) return (uint8_t)quant_store<CodeI8>(t, inv, z, g);
    if (type == LQ_U8) return (uint8_t)quant_store<CodeU8>(t, inv, z, g);
    return (uint8_t)quant_store<CodeU8S8>(t, inv, z, g);
}
__device__ __forceinline__ uint32_t nhwc_zero_code(float z, int type) {
    const int zi = (int)z;  // an integral zero point
    return (uint8_t)(type == LQ_U8S8 ? zi - 128 : zi);
}

// Epilogue of one wave's tile of 64 pixels x 16 FN channels: acc[i][j][r] is pixel
// pb + 4 j + r of this lane's run (pb = the wave's first pixel + 16 (lane / 16)), channel
// co_w + 16 i + lane % 16 of group g.  A lane owns 16 consecutive pixels of each of its FN
// channels, stored as 16-byte NCHW runs when the run lies in one image and is aligned.
constexpr int NH_ROW = 80;  // LDS bytes per channel row of the NHWC transpose (64 pixels + 16: no bank conflicts)

template <int FN, int KIND>
__device__ __forceinline__ void conv_epilogue(const ConvDmaArgs& a, v4i (&acc)[FN][4], const int pb, const int co_w,
                                              const int g, const int lane, const float* csb, const float* cbias,
                                              const int32_t* cws, const float sa, const EpiParams& ep,
                                              int8_t* nh = nullptr) {
    constexpr bool INT_CODES = KIND == LQ_OUT_Q8 || KIND == LQ_OUT_QU8 || KIND == LQ_OUT_Q16 || KIND == LQ_OUT_QU8S8;
    const int rho = lane & 15;
    const int OHW = a.OH * a.OW;
    CodeClamp cc{};
    if (INT_CODES) cc = code_clamp<KIND>(a.qmin, a.qmax);
    const int Cout = a.G * a.Cout_g;
    const int nimg = min(pb, a.P - 1) / OHW;
    const int pix0 = pb - nimg * OHW;
    constexpr int OB = OutTraits<KIND>::bytes;
    const bool vec = (OHW % 16 == 0) && (reinterpret_cast<uintptr_t>(a.y) % 16 == 0) && (pb + 15 < a.P);
    // NHWC form (nh: this wave's LDS, a row of 64 pixel bytes per channel of its tile): each
    // channel's 16-pixel run is staged as one 16-byte row segment; flush_nhwc then gives each
    // lane one pixel and reads its channels back 16 at a time, so the global stores (and the
    // skip loads of a fused residual merge) are 16 contiguous channel bytes of one pixel.
    const int cbase = g * a.Cout_g + co_w;
    // This lane's pixel of the wave's 64 in the NHWC flush, and (with a residual merge) its
    // skip codes and the merge's scalars: loaded here, before the accumulators are converted,
    // so the epilogue's arithmetic and LDS staging cover their one round trip (loaded inside
    // the flush, each 16-channel group waited for its own).
    const int fp = pb - (lane >> 4) * 16 + lane;
    int64_t fpix = 0;
    int fn = 0, foh = 0, fow = 0;
    const bool fmerge = nh != nullptr && a.skip != nullptr && fp < a.P;
    v4i sk[FN];
    float ss = 0.f, zs = 0.f, mscale = 1.f, mz = 0.f;
    if (nh != nullptr && fp < a.P) {
        fn = fp / OHW;
        const int rem = fp - fn * OHW;
        foh = rem / a.OW;
        fow = rem - foh * a.OW;
        fpix = fn * a.yimg + (int64_t)(foh + a.ypad) * a.yrow + (int64_t)(fow + a.ypad) * a.ycs;
    }
    if (fmerge) {
#pragma unroll
        for (int k = 0; k < FN; ++k)
            sk[k] = co_w + 16 * k < a.Cout_g ? *reinterpret_cast<const v4i*>(a.skip + fpix + cbase + 16 * k)
                                             : v4i{0, 0, 0, 0};
        ss = a.skip_scale[0];
        zs = a.skip_zp ? a.skip_zp[0] : 0.0f;
        mscale = a.m_scale[0];
        mz = a.m_zp ? a.m_zp[0] : 0.0f;
    }
    auto stage_nhwc = [&](const int co, const uint32_t* out) __attribute__((always_inline)) {
        v4i w;
#pragma unroll
        for (int d = 0; d < 4; ++d) w[d] = (int)pack_low_bytes(out + 4 * d);
        *reinterpret_cast<v4i*>(nh + (co - cbase) * NH_ROW + (lane >> 4) * 16) = w;
    };
    auto flush_nhwc = [&]() __attribute__((always_inline)) {
        constexpr int OT = KIND == LQ_OUT_Q8 ? LQ_I8 : KIND == LQ_OUT_QU8 ? LQ_U8 : LQ_U8S8;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (fp >= a.P) return;
        const int oh = foh, ow = fow;
        int8_t* y = static_cast<int8_t*>(a.y);
        const int64_t pix = fpix;
        const bool merge = fmerge;
        float minv = 1.f;
        Grid mg{};
        if (merge) {
            minv = 1.0f / mscale;
            mg = make_grid(a.m_qmin, a.m_qmax);
        }
        // The network's form (quint8 conv output, skip and merge, ReLU) with every scalar finite,
        // the merge zero point integral and |t * minv| below 2^21 for every t the codes can give:
        // the merge's requantize as one magic add and a med3 on the bits, as in the integer
        // epilogue (ReLU folded into the lower bound), then the shift to the stored c - 128 --
        // the same codes as quant_store.  (The shift stays a separate add: folded into the
        // rounding constant, an odd shift would move the ties-to-even.)
        bool fastm = false;
        int32_t mLm = 0, mHm = 0, mshift = 0;
        if (merge && OT == LQ_U8S8 && a.skip_type == LQ_U8S8 && a.m_type == LQ_U8S8 && a.m_relu) {
            const float bound = ((255.0f + __builtin_fabsf(ep.out_z)) * __builtin_fabsf(ep.out_s) +
                                 (255.0f + __builtin_fabsf(zs)) * __builtin_fabsf(ss)) * minv;
            fastm = minv > 0.0f && bound < 2097152.0f && mz == __builtin_rintf(mz) && __builtin_fabsf(mz) < 1048576.0f;
            if (fastm) {
                const int mzi = (int)mz;
                const int lo = min(max(mg.qlo, 0), 255), hi = max(min(mg.qhi, 255), 0);
                const int H = hi - mzi, L = min(max(lo - mzi, 0), H);
                mshift = mzi - 128;
                mLm = RNE_MAGIC_BITS + L;
                mHm = RNE_MAGIC_BITS + H;
            }
        }
        const uint32_t zc = merge ? nhwc_zero_code(mz, a.m_type) : nhwc_zero_code(ep.out_z, OT);
        const v4i zc16 = v4i{(int)(zc * 0x01010101u), (int)(zc * 0x01010101u), (int)(zc * 0x01010101u),
                             (int)(zc * 0x01010101u)};
#pragma unroll
        for (int k = 0; k < FN; ++k) {
            if (co_w + 16 * k >= a.Cout_g) break;
            const int64_t off = pix + cbase + 16 * k;
            uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int j = 0; j < 16; ++j)
                w[j >> 2] |= (uint32_t)(uint8_t)nh[(16 * k + j) * NH_ROW + (lane & 63)] << (8 * (j & 3));
            if (merge) {  // merge_bytes16_kernel's arithmetic: dequantize both, add, ReLU, requantize
                // the code types and the ReLU as constants for the common form (quint8 skip and
                // merge with ReLU: 16 values per step without per-value type tests)
                auto merge16 = [&](auto st_c, auto mt_c, auto relu_c) __attribute__((always_inline)) {
                    constexpr int ST = decltype(st_c)::value, MT = decltype(mt_c)::value;
                    constexpr int RELU = decltype(relu_c)::value;
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        uint32_t o = 0;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float av = (nhwc_code(w[d] >> (8 * e), OT) - ep.out_z) * ep.out_s;
                            const int stype = ST >= 0 ? ST : a.skip_type, mtype = MT >= 0 ? MT : a.m_type;
                            const float bv = (nhwc_code((uint32_t)sk[k][d] >> (8 * e), stype) - zs) * ss;
                            float t = av + bv;
                            if (RELU > 0 || (RELU < 0 && a.m_relu)) t = (t <= 0.0f) ? 0.0f : t;
                            o |= nhwc_store(t, minv, mz, mg, mtype) << (8 * e);
                        }
                        w[d] = o;
                    }
                };
                if (fastm) {
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        // codes c of both operands: the stored bytes c - 128 with the top bit flipped
                        const uint32_t wa = w[d] ^ 0x80808080u, wb = (uint32_t)sk[k][d] ^ 0x80808080u;
                        uint32_t o[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float av = ((float)((wa >> (8 * e)) & 0xffu) - ep.out_z) * ep.out_s;
                            const float bv = ((float)((wb >> (8 * e)) & 0xffu) - zs) * ss;
                            const float t = av + bv;
                            o[e] = (uint32_t)(med3_i32(rne_bits(t * minv), mLm, mHm) + mshift);
                        }
                        w[d] = pack_low_bytes(o);
                    }
                } else if (a.skip_type == LQ_U8S8 && a.m_type == LQ_U8S8 && a.m_relu)
                    merge16(std::integral_constant<int, LQ_U8S8>{}, std::integral_constant<int, LQ_U8S8>{},
                            std::integral_constant<int, 1>{});
                else
                    merge16(std::integral_constant<int, -1>{}, std::integral_constant<int, -1>{},
                            std::integral_constant<int, -1>{});
            }
            *reinterpret_cast<v4i*>(y + off) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
            if (a.ypad) {
                const bool l = ow == 0, r = ow == a.OW - 1;
                const int64_t cs = a.ycs, rw = a.yrow;
                if (l) *reinterpret_cast<v4i*>(y + off - cs) = zc16;
                if (r) *reinterpret_cast<v4i*>(y + off + cs) = zc16;
                if (oh == 0) {
                    *reinterpret_cast<v4i*>(y + off - rw) = zc16;
                    if (l) *reinterpret_cast<v4i*>(y + off - rw - cs) = zc16;
                    if (r) *reinterpret_cast<v4i*>(y + off - rw + cs) = zc16;
                }
                if (oh == a.OH - 1) {
                    *reinterpret_cast<v4i*>(y + off + rw) = zc16;
                    if (l) *reinterpret_cast<v4i*>(y + off + rw - cs) = zc16;
                    if (r) *reinterpret_cast<v4i*>(y + off + rw + cs) = zc16;
                }
            }
        }
    };
    // Stores of one channel's 16 consecutive pixels (out[] holds the output type's bits).
    auto store_col = [&](const int co, const uint32_t* out) __attribute__((always_inline)) {
        if constexpr (OB == 1) {
            if (nh) {
                stage_nhwc(co, out);
                return;
            }
        }
        if (vec) {
            const int64_t base = ((int64_t)nimg * Cout + co) * OHW + pix0;
            if (OB == 1) {
                v4i w;
#pragma unroll
                for (int d = 0; d < 4; ++d) w[d] = (int)pack_low_bytes(out + 4 * d);
                *reinterpret_cast<v4i*>(reinterpret_cast<uint8_t*>(a.y) + base) = w;
            } else if (OB == 2) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    v4i w;
#pragma unroll
                    for (int d = 0; d < 4; ++d)
                        w[d] = (int)((out[8 * h + 2 * d] & 0xffffu) | (out[8 * h + 2 * d + 1] << 16));
                    *reinterpret_cast<v4i*>(reinterpret_cast<uint16_t*>(a.y) + base + 8 * h) = w;
                }
            } else {
#pragma unroll
                for (int h = 0; h < 4; ++h)
                    *reinterpret_cast<v4i*>(reinterpret_cast<uint32_t*>(a.y) + base + 4 * h) =
                        v4i{(int)out[4 * h], (int)out[4 * h + 1], (int)out[4 * h + 2], (int)out[4 * h + 3]};
            }
        } else {
            // 16 consecutive pixels from (image nimg, pixel pix0): at most one image boundary
            // when OHW >= 16 (else the division per pixel)
            const int64_t base = ((int64_t)nimg * Cout + co) * OHW + pix0;
            const int64_t next = ((int64_t)(nimg + 1) * Cout + co) * OHW + pix0 - OHW;
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int p = pb + q;
                if (p >= a.P) break;
                int64_t idx;
                if (OHW >= 16) {
                    idx = pix0 + q < OHW ? base + q : next + q;
                } else {
                    const int nq = p / OHW, pq = p - nq * OHW;
                    idx = ((int64_t)nq * Cout + co) * OHW + pq;
                }
                store_elem<KIND>(a.y, idx, out[q]);
            }
        }
    };

    // Integer codes, fast form (as in the GEMM epilogue): with the output scale's reciprocal
    // finite and positive, the zero point integral and small, and every scale and bias of this
    // wave finite and small enough that y stays finite, clamp(rne(y * inv) + z, lo, hi) equals
    // zi + med3(rne(y * inv), lo - zi, hi - zi), the rounding and clamp on rne_bits against
    // bounds shifted by RNE_MAGIC_BITS (|zi| < 2^21), and ReLU folds into the lower bound.
    if constexpr (INT_CODES) {
        const float zf = ep.out_z;
        bool ok = ep.out_inv > 0.0f && ep.out_inv < 3.0e38f && zf == __builtin_rintf(zf) &&
                  __builtin_fabsf(zf) < 2097152.0f && __builtin_isfinite(sa);
        float bmax = 0.0f;
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            bmax = __builtin_fmaxf(bmax, __builtin_fabsf(csb[i]));
            ok = ok && __builtin_isfinite(csb[i]) && __builtin_isfinite(cbias[i]);
        }
        const float amax = __builtin_fabsf(sa);
        ok = ok && amax < 1.0e14f && bmax < 1.0e14f && amax * bmax < 1.0e28f;
        if (__all(ok)) {
            const int zi = (int)zf;
            int L = cc.lo - zi, H = cc.hi - zi;
            if (a.relu) L = max(L, 0);
            L = min(L, H);  // med3(x, L, H) = min(max(x, L), H) needs L <= H
            const int Lm = L + RNE_MAGIC_BITS, Hm = H + RNE_MAGIC_BITS;
            const int shift = zi - (KIND == LQ_OUT_QU8S8 ? 128 : 0);
            auto cols = [&](auto bias_c, auto za_c, auto shift_c) __attribute__((always_inline)) {
                constexpr bool BIAS = decltype(bias_c)::value, ZA = decltype(za_c)::value;
                constexpr bool SHIFT = decltype(shift_c)::value;
                static_for<FN>([&](auto i_c) __attribute__((always_inline)) {
                    constexpr int i = decltype(i_c)::value;
                    const int col = co_w + 16 * i + rho;
                    if (col >= a.Cout_g) return;
                    const float sc = sa * csb[i];
                    const uint32_t zsum = (uint32_t)ep.za * (uint32_t)cws[i];
                    uint32_t out[16];
#pragma unroll
                    for (int q = 0; q < 16; ++q) {
                        int32_t accq = acc[i][q >> 2][q & 3];
                        if (ZA) accq = (int32_t)((uint32_t)accq - zsum);
                        float y = (float)accq * sc;
                        if (BIAS) y = y + cbias[i];
                        int32_t c = med3_i32(rne_bits(y * ep.out_inv), Lm, Hm);
                        if (SHIFT) c += shift;
                        out[q] = (uint32_t)c;  // low byte / halfword: the code
                    }
                    store_col(g * a.Cout_g + col, out);
                });
            };
            auto cols_za = [&](auto bias_c) __attribute__((always_inline)) {
                if (ep.has_za) {
                    if (shift != 0) cols(bias_c, std::true_type{}, std::true_type{});
                    else cols(bias_c, std::true_type{}, std::false_type{});
                } else {
                    if (shift != 0) cols(bias_c, std::false_type{}, std::true_type{});
                    else cols(bias_c, std::false_type{}, std::false_type{});
                }
            };
            if (a.bias) cols_za(std::true_type{});
            else cols_za(std::false_type{});
            if constexpr (OB == 1) {
                if (nh) flush_nhwc();
            }
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < FN; ++i) {
        const int col = co_w + 16 * i + rho;
        if (col >= a.Cout_g) continue;
        const int co = g * a.Cout_g + col;
        const float sb = csb[i];
        const float bias = cbias[i];
        const int32_t zsum = ep.has_za ? (int32_t)((uint32_t)ep.za * (uint32_t)cws[i]) : 0;
        uint32_t out[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int32_t acc_c = (int32_t)((uint32_t)acc[i][q >> 2][q & 3] - (uint32_t)zsum);
            if (INT_CODES) {
                const float s = sa * sb;
                float y = (float)acc_c * s;
                if (a.bias) y = y + bias;
                if (a.relu) y = (y <= 0.0f) ? 0.0f : y;
                out[q] = (uint32_t)requant_int<KIND>(y, ep, cc);
                if (KIND == LQ_OUT_QU8S8) out[q] ^= 0x80u;
            } else {
                out[q] = epi_one<KIND>(acc_c, sa, sb, a.bias ? &bias : nullptr, a.relu != 0, ep);
            }
        }
        store_col(co, out);
    }
    if constexpr (OB == 1) {
        if (nh) flush_nhwc();
    }
}

// ---------------------------------------------------------------- halo-staged direct conv
//
// Stride-1, zeros-padded, undilated, ungrouped convolutions with 64 input channels, Cout a
// multiple of 64 and H * W a multiple of 16 (ResNet-18 layer1) skip the padded NHWC copy.  A
// workgroup of four waves owns 256 consecutive output pixels (flattened n, oh, ow) x 64 output
// channels.  For each block of 64 input channels it stages in LDS
//   * the halo: every padded input row its pixels read -- padded rows of consecutive images
//     stack, row R = n * Hp + hp, and the tile needs rows R0 .. R0 + HR - 1 -- at all Wp padded
//     columns, 64 channels per position (64 bytes; 16-byte chunk c at slot c ^ ((pos >> 4) & 3),
//     which spreads the four 4-pixel runs of an A fragment over distinct banks), read from the
//     NCHW codes as 16-byte chunks of each channel's contiguous run of rows and transposed 4 x 4
//     in registers (v_perm); padding positions and rows past the last image hold the
//     activation zero point;
//   * the block's weights for the 64 output channels, [tap][co][64 bytes] (chunk slot
//     c ^ ((co >> 2) & 3)), by LDS-DMA from the packed rows;
// then runs every tap from LDS: tap (kh, kw) of pixel (n, oh, ow) is halo position
// (n * Hp + oh + kh - R0) * Wp + ow + kw.  Each staged input byte serves all KH * KW taps and
// no padded copy of the activation goes through HBM.  Pixels are the MFMA row operand in the
// permuted order of the DMA kernel (a lane ends with 16 consecutive pixels of each of its
// channels), so the epilogue is the same.
constexpr int CV_HALO_ITEMS = 3;  // staged 4-channel x 16-byte items per thread per image

struct HaloArgs {
    ConvDmaArgs e;      // output, geometry (P, OH, OW, Cout_g, G = 1), epilogue operands
    const int8_t* x;    // NCHW activation codes
    int N, C, H, W, Hp, Wp, pt, pl, KH, KW, nc;  // nc = C / 64 input channel blocks
    int halo_bytes;     // LDS bytes of the largest tile's halo (a multiple of 1024)
    float inv_ohw, inv_ow, inv_hp, inv_w;  // 1 / (OH * OW), 1 / OW, 1 / Hp, 1 / W (div_small)
    int dummy_pos;      // halo position past the last row: a sink for bytes outside the run
};

__device__ __forceinline__ int halo_slot(int pos, int chunk) { return chunk ^ ((pos >> 4) & 3); }

// q / d for 0 <= q < 2^24 and d >= 1 by a float reciprocal estimate (within one of the quotient
// for such q) and one correction each way: a handful of VALU ops where an integer division
// by a runtime value is a long sequence.
__device__ __forceinline__ int div_small(int q, int d, float inv) {
    int n = (int)((float)q * inv);
    n -= (n * d > q) ? 1 : 0;
    n += ((n + 1) * d <= q) ? 1 : 0;
    return n;
}

template <int KIND>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void conv_i8_halo_kernel(HaloArgs h) {
    const ConvDmaArgs& a = h.e;
    extern __shared__ __attribute__((aligned(1024))) int8_t halo_lds[];
    int8_t* hal = halo_lds;
    const int8_t* wl = halo_lds + h.halo_bytes;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int p0 = blockIdx.x * 256, co0 = blockIdx.y * 64;
    const int OHW = a.OH * a.OW, T = h.KH * h.KW;
    // padded rows of this tile (stride 1: output row oh reads padded rows oh .. oh + KH - 1)
    const int plast = min(p0 + 255, a.P - 1);
    const int n0 = div_small(p0, OHW, h.inv_ohw), oh0 = div_small(p0 - n0 * OHW, a.OW, h.inv_ow);
    const int n1 = div_small(plast, OHW, h.inv_ohw), oh1 = div_small(plast - n1 * OHW, a.OW, h.inv_ow);
    const int R0 = n0 * h.Hp + oh0;
    const int HR = n1 * h.Hp + oh1 + h.KH - R0;

    // epilogue operands (the oldest loads: the staging waits cover them)
    const int rho = lane & 15, c0 = lane >> 4;
    float csb[4], cbias[4];
    int32_t cws[4];
    EpiParams ep;
    ep.za = (a.a_zp ? (int)a.a_zp[0] : 0) - (a.a_u8s8 ? 128 : 0);
    ep.has_za = a.a_zp != nullptr || a.a_u8s8;
    ep.out_s = a.out_scale ? a.out_scale[0] : 1.0f;
    ep.out_inv = 1.0f / ep.out_s;
    ep.out_z = a.out_zp ? a.out_zp[0] : 0.0f;
    ep.g = make_grid(a.qmin, a.qmax);
    const float sa = a.a_scale ? a.a_scale[0] : 1.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int co = min(co0 + 16 * i + rho, a.Cout_g - 1);
        csb[i] = a.w_scale[co];
        cbias[i] = a.bias ? a.bias[co] : 0.0f;
        cws[i] = ep.has_za ? a.w_sums[co] : 0;
    }
    const uint32_t fill8 = (uint32_t)(uint8_t)(int8_t)ep.za;
    const uint32_t fill = fill8 * 0x01010101u;

    // halo position of tap (0, 0) for the four pixels of this lane's A fragments
    int basepos[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int q = min(p0 + wave * 64 + (rho >> 2) * 16 + 4 * j + (rho & 3), a.P - 1);
        const int n = div_small(q, OHW, h.inv_ohw), r = q - n * OHW;
        const int oh = div_small(r, a.OW, h.inv_ow), ow = r - oh * a.OW;
        basepos[j] = (n * h.Hp + oh - R0) * h.Wp + ow;
    }

    const v4i rw = buffer_rsrc(a.wp, (uint32_t)((int64_t)a.Cout_g * a.ldw));
    const uint32_t wl_base = (uint32_t)reinterpret_cast<uintptr_t>(wl);
    const int side = h.Wp - h.W;                 // padding columns per row
    const int nA = div_small(R0, h.Hp, h.inv_hp), nB = min(div_small(R0 + HR - 1, h.Hp, h.inv_hp), h.N - 1);
    v4i acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    for (int cb = 0; cb < h.nc; ++cb) {
        if (cb > 0) block_barrier();  // every wave is done reading the previous block
        // weights of this channel block: row (tap, co) of 64 bytes, 16 rows per copy
        for (int i = wave; i < T * 4; i += 4) {
            const int row = i * 16 + (lane >> 2);
            const int tap = row >> 6, co = row & 63;
            const int chunk = (lane & 3) ^ ((co >> 2) & 3);
            const uint32_t off = (uint32_t)((co0 + co) * a.ldw + tap * h.C + cb * 64 + chunk * 16);
            lds_dma16(rw, off, 0, wl_base + (uint32_t)i * 1024u);
        }
        // halo interior, image by image: the tile's input rows ihA..ihB of image n are one
        // contiguous run of bytes in each channel plane.  Work item = (channel quad cq, 16-byte
        // chunk k of the run), k fastest so a wave's loads run along channel planes; a thread
        // loads its items' 4 x 16 bytes (4 channels) first, then transposes each column of 4
        // channel bytes into a dword (v_perm) and writes it at its halo position.  Bytes of a
        // chunk outside the run (alignment) go to a dummy slot past the halo.
        for (int n = nA; n <= nB; ++n) {
            const int hpA = max(R0 - n * h.Hp, 0), hpB = min(R0 + HR - 1 - n * h.Hp, h.Hp - 1);
            const int ihA = max(hpA - h.pt, 0), ihB = min(hpB - h.pt, h.H - 1);
            if (ihA > ihB) continue;
            const int b0 = ihA * h.W, b1 = (ihB + 1) * h.W;  // byte range of the run in a plane
            const int kA = b0 >> 4, nk = ((b1 - 1) >> 4) - kA + 1;
            const int items = nk * 16;
            const int rowbase = n * h.Hp + h.pt - R0;  // halo row of input row 0 of image n
            const int8_t* plane0 = h.x + ((int64_t)n * h.C + cb * 64) * h.H * h.W;
            constexpr int IT = CV_HALO_ITEMS;
            v4i d[IT][4];
            int kk[IT], cq[IT];
#pragma unroll
            for (int b = 0; b < IT; ++b) {
                const int it = min(tid + b * 256, items - 1);
                cq[b] = div_small(it, nk, __builtin_amdgcn_rcpf((float)nk));
                kk[b] = kA + it - cq[b] * nk;
                const int8_t* src = plane0 + (int64_t)(4 * cq[b]) * h.H * h.W + 16 * kk[b];
#pragma unroll
                for (int t = 0; t < 4; ++t) d[b][t] = *reinterpret_cast<const v4i*>(src + (int64_t)t * h.H * h.W);
            }
#pragma unroll
            for (int b = 0; b < IT; ++b) {
                if (tid + b * 256 >= items) continue;
                const int j0 = 16 * kk[b];
                int ih = div_small(j0, h.W, h.inv_w), col = j0 - ih * h.W;
#pragma unroll
                for (int q = 0; q < 4; ++q) {  // dword q of each channel: columns 4 q .. 4 q + 3
                    const uint32_t t01l = __builtin_amdgcn_perm(d[b][1][q], d[b][0][q], 0x05010400u);
                    const uint32_t t01h = __builtin_amdgcn_perm(d[b][1][q], d[b][0][q], 0x07030602u);
                    const uint32_t t23l = __builtin_amdgcn_perm(d[b][3][q], d[b][2][q], 0x05010400u);
                    const uint32_t t23h = __builtin_amdgcn_perm(d[b][3][q], d[b][2][q], 0x07030602u);
                    const uint32_t o[4] = {__builtin_amdgcn_perm(t23l, t01l, 0x05040100u),
                                           __builtin_amdgcn_perm(t23l, t01l, 0x07060302u),
                                           __builtin_amdgcn_perm(t23h, t01h, 0x05040100u),
                                           __builtin_amdgcn_perm(t23h, t01h, 0x07060302u)};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int j = j0 + 4 * q + e;
                        const int pos = (j >= b0 && j < b1) ? (rowbase + ih) * h.Wp + h.pl + col : h.dummy_pos;
                        *reinterpret_cast<uint32_t*>(hal + pos * 64 + (halo_slot(pos, cq[b] >> 2) << 4) + (cq[b] & 3) * 4) = o[e];
                        if (++col == h.W) col = 0, ++ih;
                    }
                }
            }
        }
        // fill code: every position of a halo row outside the images, the padding columns of
        // the others (16-byte chunks)
        for (int r = 0; r < HR; ++r) {
            const int R = R0 + r, n = div_small(R, h.Hp, h.inv_hp), hp = R - n * h.Hp;
            const bool inside = n < h.N && hp >= h.pt && hp < h.pt + h.H;
            const int cells = inside ? side : h.Wp;
            for (int v = tid; v < cells * 4; v += 256) {
                const int chunk = v & 3, k = v >> 2;
                const int wp = inside ? (k < h.pl ? k : h.W + k) : k;
                const int pos = r * h.Wp + wp;
                *reinterpret_cast<v4i*>(hal + pos * 64 + (halo_slot(pos, chunk) << 4)) =
                    v4i{(int)fill, (int)fill, (int)fill, (int)fill};
            }
        }
        wait_vmcnt<0>();
        block_barrier();

        // every tap from LDS; fragments of tap t + 1 are read while tap t's MFMAs run
        auto read_frags = [&](v4i* f, int t) __attribute__((always_inline)) {
            const int kh = t / h.KW, kw = t - kh * h.KW;
            const int toff = kh * h.Wp + kw;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int pos = basepos[j] + toff;
                f[j] = *reinterpret_cast<const v4i*>(hal + pos * 64 + (halo_slot(pos, c0) << 4));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int co = 16 * i + rho;
                f[4 + i] = *reinterpret_cast<const v4i*>(wl + (t * 64 + co) * 64 + ((c0 ^ ((co >> 2) & 3)) << 4));
            }
        };
        auto mfmas = [&](const v4i* f) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(f[j], f[4 + i], acc[i][j], 0, 0, 0);
        };
        v4i F0[8], F1[8];
        read_frags(F0, 0);
        int t = 0;
        for (; t + 2 <= T; t += 2) {
            read_frags(F1, t + 1);
            mfmas(F0);
            if (t + 2 < T) read_frags(F0, t + 2);
            mfmas(F1);
        }
        if (t < T) mfmas(F0);
    }
    conv_epilogue<4, KIND>(a, acc, p0 + wave * 64 + c0 * 16, co0, 0, lane, csb, cbias, cws, sa, ep);
}

// Halo plan: the largest halo over the tiles (exact, by walking the tile starts), or 0 when
// the shape does not take the halo kernel.
constexpr int CV_HALO_LDS = 80 * 1024;  // two workgroups per CU
int64_t halo_bytes_for(int64_t N, int64_t C, int64_t H, int64_t W, int64_t Cout, int64_t KH, int64_t KW, int sh,
                       int sw, int pt, int pb, int pl, int pr, int dh, int dw, int64_t groups, int mode, int64_t OH,
                       int64_t OW) {
    if (groups != 1 || sh != 1 || sw != 1 || dh != 1 || dw != 1 || mode != LQ_PAD_ZEROS) return 0;
    // (W <= 64: the 16 channel quads x W / 4 column quads of a row fit the 256 threads)
    // One block of 64 input channels: with more, the single-buffered staging of each block is
    // exposed (ResNet layer2, C = 128: 21.8 us against 19.0 us for the packed-input kernel).
    if (C != 64 || Cout % 64 != 0 || (H * W) % 16 != 0 || KH * KW > 16) return 0;
    const int64_t Hp = H + pt + pb, Wp = W + pl + pr, OHW = OH * OW, P = N * OHW;
    if (OHW < 64 || P < 256 || N * Hp >= (1 << 24) || P >= (1 << 24)) return 0;
    int64_t hr = 0;
    for (int64_t p0 = 0; p0 < P; p0 += 256) {
        const int64_t last = std::min(p0 + 255, P - 1);
        const int64_t n0 = p0 / OHW, oh0 = (p0 - n0 * OHW) / OW;
        const int64_t n1 = last / OHW, oh1 = (last - n1 * OHW) / OW;
        const int64_t R0 = n0 * Hp + oh0, R1 = n1 * Hp + oh1 + KH - 1;
        hr = std::max(hr, R1 - R0 + 1);
        // per image, the run of input rows must fit CV_HALO_ITEMS items per thread
        for (int64_t n = R0 / Hp; n <= std::min(R1 / Hp, N - 1); ++n) {
            const int64_t ihA = std::max<int64_t>(std::max<int64_t>(R0 - n * Hp, 0) - pt, 0);
            const int64_t ihB = std::min<int64_t>(std::min<int64_t>(R1 - n * Hp, Hp - 1) - pt, H - 1);
            if (ihA > ihB) continue;
            const int64_t nk = ((ihB + 1) * W - 1) / 16 - (ihA * W) / 16 + 1;
            if (nk * 16 > CV_HALO_ITEMS * 256) return 0;
        }
    }
    const int64_t bytes = (hr * Wp * 64 + 1023) / 1024 * 1024 + 1024;  // + the dummy position
    if (bytes + KH * KW * 4096 > CV_HALO_LDS) return 0;
    return bytes;
}

// Two waves per SIMD (<= 256 registers): the LDS ring leaves room for two workgroups per CU,
// and their main loops and epilogues overlap.
// KSPLIT > 1 (NHWC, one K range per workgroup): KSPLIT groups of WAVES_M x WAVES_N waves, each
// with its own stage ring, run equal shares of the K stages side by side; the groups' exact
// int32 tile sums meet in LDS and group 0 runs the epilogue -- the waves of a cross-workgroup
// split without its second launch.
template <int BM, int BN, int WAVES_M, int WAVES_N, int NBUF, int KIND, bool NHWC = false, int KSPLIT = 1>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N * KSPLIT) __attribute__((amdgpu_waves_per_eu(2))) void conv_i8_dma_kernel(
    ConvDmaArgs a) {
    constexpr int BK = 128, NW = WAVES_M * WAVES_N, WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int FM = WM / 16, FN = WN / 16;
    constexpr int A_I = BM / 8 / NW, B_I = BN / 8 / NW, LPS = A_I + B_I, SB = (BM + BN) * BK;
    static_assert(WM == 64, "a lane owns 16 consecutive pixels of a 64-pixel wave tile");
    static_assert(A_I * 8 * NW == BM && B_I * 8 * NW == BN && WN % 16 == 0, "copy split");
    static_assert(NBUF >= 2 && (NBUF - 1) * LPS < 64, "stage ring");
    static_assert(KSPLIT == 1 || NHWC, "the in-workgroup K split serves the NHWC form");
    static_assert(KSPLIT * NBUF * SB <= 160 * 1024, "LDS budget");
    __shared__ __attribute__((aligned(1024))) int8_t lds_all[KSPLIT * NBUF * SB];

    const int p0 = blockIdx.x * BM, co0 = blockIdx.y * BN;
    const int split = a.phase == 0 ? (int)blockIdx.z % a.splits : 0;
    const int g = a.phase == 0 ? (int)blockIdx.z / a.splits : (int)blockIdx.z;
    const int lane = threadIdx.x & 63;
    const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kgrp = wave_all / NW;     // this wave's K group (0 when KSPLIT == 1)
    const int wave = wave_all % NW;     // its wave within the group's tile layout
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    int8_t* const lds = lds_all + kgrp * NBUF * SB;  // the group's stage ring
    const int GCp = a.G * a.Cp;
    // K stages of this split: [kb, kb + nks); with KSPLIT the group's equal share of them
    // (the host takes KSPLIT > 1 only when it divides the stage count)
    const int per_split = (a.nk + a.splits - 1) / a.splits;
    const int kb = split * per_split + kgrp * (min(a.nk - split * per_split, per_split) / KSPLIT);
    const int nks = min(a.nk - split * per_split, per_split) / KSPLIT;
    // this tile's partial sums: splits x (FN x FM fragments) x (threads) int32x4, thread-minor
    constexpr int NFRAG = FN * FM;
    const int64_t tile_lin = ((int64_t)g * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    v4i* part = reinterpret_cast<v4i*>(a.part) + tile_lin * a.splits * NFRAG * (64 * NW) + threadIdx.x;
    const int taps = a.KH * a.KW;
    // input offset of tap t (the K padding past KH * KW reads tap 0; its weights are zero)
    auto tap_off = [&](int t) __attribute__((always_inline)) {
        const int kh = (t * a.kw_magic) >> 16, kw = t - kh * a.KW;
        return t < taps ? kh * a.kh_stride + kw * a.kw_stride : 0;
    };

    const v4i rx = buffer_rsrc(a.xp, a.xp_bytes);
    const v4i rw = buffer_rsrc(a.wp + (int64_t)g * a.Cout_g * a.ldw, (uint32_t)((int64_t)a.Cout_g * a.ldw));
    const int rl = lane >> 3, slot = lane & 7;
    const int OHW = a.OH * a.OW;
    uint32_t abase[A_I];
    int aq[A_I];  // logical 16-byte chunk of the lane's copy (the swizzle is per row)
#pragma unroll
    for (int j = 0; j < A_I; ++j) {
        const int r = (j * NW + wave) * 8 + rl;
        const int p = min(p0 + r, a.P - 1);
        const int n = p / OHW, rem = p - n * OHW;
        const int oh = rem / a.OW, ow = rem - oh * a.OW;
        abase[j] = (uint32_t)((((int64_t)n * a.Hp + (int64_t)oh * a.sh) * a.Wp + (int64_t)ow * a.sw) * GCp +
                              (int64_t)g * a.Cp);
        aq[j] = slot ^ dma_swz(r);
    }
    uint32_t boff[B_I];
#pragma unroll
    for (int j = 0; j < B_I; ++j) {
        const int r = (j * NW + wave) * 8 + rl;
        boff[j] = (uint32_t)((co0 + r) * a.ldw + (slot ^ dma_swz(r)) * 16);
    }
    const uint32_t lds_base = (uint32_t)reinterpret_cast<uintptr_t>(lds);
    auto issue = [&](int buf, int kt) __attribute__((always_inline)) {
        const int k0 = (kb + min(kt, nks - 1)) * BK;
        const uint32_t sb = lds_base + buf * SB;
        const int tap_u = a.cp_shift < 0 ? k0 / a.Cp : 0;  // Cp a multiple of 128: one tap per stage
#pragma unroll
        for (int j = 0; j < A_I; ++j) {
            const int k = k0 + 16 * aq[j];
            const int tap = a.cp_shift < 0 ? tap_u : (k >> a.cp_shift);
            const uint32_t off = abase[j] + (uint32_t)(tap_off(tap) + (k - tap * a.Cp));
            lds_dma16(rx, off, 0, sb + (j * NW + wave) * 8 * BK);
        }
#pragma unroll
        for (int j = 0; j < B_I; ++j) lds_dma16(rw, boff[j], (uint32_t)k0, sb + BM * BK + (j * NW + wave) * 8 * BK);
    };
    // Fragments: pixel fragment j (permuted rows wm*64 + (rho/4)*16 + 4j + rho%4), channel
    // fragment i (rows wn*WN + 16 i + rho); logical chunk of K step s: 4 s + lane / 16.
    const int rho = lane & 15, c0 = lane >> 4;
    const int a_row = wm * 64 + (rho >> 2) * 16 + (rho & 3);
    const int a_base = a_row * BK + ((c0 ^ dma_swz(a_row)) << 4);
    const int b_base = BM * BK + (wn * WN + rho) * BK + ((c0 ^ (rho & 7)) << 4);
    v4i F0[FM + FN], F1[FM + FN];
    auto read_frags = [&](v4i* f, int buf, int s) __attribute__((always_inline)) {
        const int8_t* sbuf = lds + buf * SB;
#pragma unroll
        for (int j = 0; j < FM; ++j)
            f[j] = *reinterpret_cast<const v4i*>(sbuf + (a_base ^ (((s ^ j) & 1) << 6)) + j * 4 * BK);
#pragma unroll
        for (int i = 0; i < FN; ++i)
            f[FM + i] = *reinterpret_cast<const v4i*>(sbuf + (b_base ^ (((s ^ i) & 1) << 6)) + i * 16 * BK);
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
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(f[j], f[FM + i], acc[i][j], 0, 0, 0);
    };
    // A ring of NBUF stage buffers: NBUF stages are issued up front; at stage kt the wait
    // leaves stages kt+2 .. kt+NBUF-1 in flight, and after the barrier (every wave's reads of
    // buffer kt done) stage kt+NBUF is issued into it.  Stages past the end are clamped to the
    // last (a valid address, landing in a buffer never read again), so the counts are static.
    auto stage = [&](auto bc, int kt, bool last) __attribute__((always_inline)) {
        constexpr int B = decltype(bc)::value;
        read_frags(F1, B, 1);
        mfmas(F0);
        if (!last) {
            wait_vmcnt<(NBUF - 2) * LPS>();
            block_barrier();
            issue(B, kt + NBUF);
            read_frags(F0, (B + 1) % NBUF, 0);
        }
        mfmas(F1);
    };
    // Epilogue inputs of this lane's FN channels, loaded before the main loop so their latency
    // hides under it (they are the oldest loads: the stage waits cover them).
    const int rho_e = lane & 15;
    float csb[FN], cbias[FN];
    int32_t cws[FN];
    const bool epilogue_here = a.phase == 1 || a.splits == 1;
    // the per-call scalars too (their loads and the reciprocal would otherwise open the
    // epilogue with a memory round trip)
    EpiParams ep;
    ep.za = (a.a_zp ? (int)a.a_zp[0] : 0) - (a.a_u8s8 ? 128 : 0);
    ep.has_za = a.a_zp != nullptr || a.a_u8s8;
    ep.out_s = a.out_scale ? a.out_scale[0] : 1.0f;
    ep.out_inv = 1.0f / ep.out_s;
    ep.out_z = a.out_zp ? a.out_zp[0] : 0.0f;
    ep.g = make_grid(a.qmin, a.qmax);
    const float sa = a.a_scale ? a.a_scale[0] : 1.0f;
    if (epilogue_here) {
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            const int col = min(co0 + wn * WN + 16 * i + rho_e, a.Cout_g - 1);
            const int co = g * a.Cout_g + col;
            csb[i] = a.w_scale[co];
            cbias[i] = a.bias ? a.bias[co] : 0.0f;
            cws[i] = (a.a_zp != nullptr || a.a_u8s8) ? a.w_sums[co] : 0;
        }
    }
    if (a.phase == 1) {
        // the splits' exact sums, added in split order (int32 wrap-around: any order gives the
        // same bits)
#pragma unroll
        for (int sp = 0; sp < a.splits; ++sp)
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j) {
                    const v4i v = part[((int64_t)sp * NFRAG + i * FM + j) * (64 * NW)];
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][j][r] = (int)((uint32_t)acc[i][j][r] + (uint32_t)v[r]);
                }
    } else {
#pragma unroll
        for (int j = 0; j < NBUF; ++j) issue(j, j);
        wait_vmcnt<(NBUF - 1) * LPS>();
        block_barrier();
        read_frags(F0, 0, 0);
        int kt = 0;
        for (; kt + NBUF < nks; kt += NBUF) {
            [&]<int... B>(std::integer_sequence<int, B...>) {
                (stage(std::integral_constant<int, B>(), kt + B, false), ...);
            }(std::make_integer_sequence<int, NBUF>());
        }
        [&]<int... B>(std::integer_sequence<int, B...>) {
            ((kt + B < nks ? stage(std::integral_constant<int, B>(), kt + B, kt + B + 1 == nks) : void()), ...);
        }(std::make_integer_sequence<int, NBUF>());
        wait_vmcnt<0>();  // no copy may still target LDS when the workgroup ends
        if (a.splits > 1) {
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j) part[((int64_t)split * NFRAG + i * FM + j) * (64 * NW)] = acc[i][j];
            return;
        }
    }

    if constexpr (NHWC) {
        // the transpose reuses the stage ring once every wave is done reading it (a separate
        // array would cost the second workgroup per CU)
        static_assert(NW * WN * NH_ROW <= NBUF * SB, "NHWC transpose in the stage ring");
        block_barrier();
        if constexpr (KSPLIT > 1) {
            // groups 1.. leave their tile sums past group 0's transpose rows; group 0 adds them
            // (int32 wrap-around: any order gives the same bits) and runs the epilogue
            constexpr int RED_OFF = (NW * WN * NH_ROW + 1023) / 1024 * 1024;
            static_assert(RED_OFF + (KSPLIT - 1) * NFRAG * 64 * NW * 16 <= KSPLIT * NBUF * SB, "tile sums in LDS");
            v4i* red = reinterpret_cast<v4i*>(lds_all + RED_OFF);
            if (kgrp > 0) {
#pragma unroll
                for (int i = 0; i < FN; ++i)
#pragma unroll
                    for (int j = 0; j < FM; ++j)
                        red[(((kgrp - 1) * NFRAG + i * FM + j) * NW + wave) * 64 + lane] = acc[i][j];
            }
            block_barrier();
            if (kgrp > 0) return;  // no barrier follows
#pragma unroll
            for (int gq = 1; gq < KSPLIT; ++gq)
#pragma unroll
                for (int i = 0; i < FN; ++i)
#pragma unroll
                    for (int j = 0; j < FM; ++j) {
                        const v4i v = red[(((gq - 1) * NFRAG + i * FM + j) * NW + wave) * 64 + lane];
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[i][j][r] = (int)((uint32_t)acc[i][j][r] + (uint32_t)v[r]);
                    }
        }
        conv_epilogue<FN, KIND>(a, acc, p0 + wm * 64 + c0 * 16, co0 + wn * WN, g, lane, csb, cbias, cws, sa, ep,
                                lds_all + wave * WN * NH_ROW);
    } else {
        conv_epilogue<FN, KIND>(a, acc, p0 + wm * 64 + c0 * 16, co0 + wn * WN, g, lane, csb, cbias, cws, sa, ep);
    }
}

// ---------------------------------------------------------------- float helpers

struct FConvArgs {
    const float* x;
    const float* w;
    const float* bias;
    float* y;
    int N, C, H, W, Cout, G, Cg, Cout_g, KH, KW, sh, sw, pt, pl, dh, dw, OH, OW, mode;
};

// Direct float convolution, one thread per output: sum over (c, kh, kw) in that order,
// float32 multiply then add (no FMA), bias added last.
__global__ __launch_bounds__(256) void conv_f32_kernel(FConvArgs a) {
    const int64_t total = (int64_t)a.N * a.Cout * a.OH * a.OW;
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= total) return;
    const int ow = (int)(id % a.OW);
    int64_t r = id / a.OW;
    const int oh = (int)(r % a.OH);
    r /= a.OH;
    const int co = (int)(r % a.Cout);
    const int n = (int)(r / a.Cout);
    const int g = co / a.Cout_g;
    float acc = 0.0f;
    for (int c = 0; c < a.Cg; ++c) {
        const float* xc = a.x + ((int64_t)n * a.C + (int64_t)g * a.Cg + c) * a.H * a.W;
        const float* wc = a.w + ((int64_t)co * a.Cg + c) * a.KH * a.KW;
        for (int kh = 0; kh < a.KH; ++kh) {
            const int h = pad_index(oh * a.sh + kh * a.dh - a.pt, a.H, a.mode);
            if (h < 0) continue;
            for (int kw = 0; kw < a.KW; ++kw) {
                const int w = pad_index(ow * a.sw + kw * a.dw - a.pl, a.W, a.mode);
                if (w < 0) continue;
                const float prod = xc[(int64_t)h * a.W + w] * wc[kh * a.KW + kw];
                acc = acc + prod;
            }
        }
    }
    if (a.bias) acc = acc + a.bias[co];
    a.y[id] = acc;
}

// Eval BatchNorm over NCHW: y = fl32(fl32(fl32(x - mean) * fl32(1 / sqrt(var + eps))) * gamma) + beta.
__global__ __launch_bounds__(256) void batch_norm_f32_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                             int64_t N, int C, int64_t HW, const float* __restrict__ mean,
                                                             const float* __restrict__ var, const float* __restrict__ gamma,
                                                             const float* __restrict__ beta, float eps) {
    const int64_t total = N * C * HW;
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= total) return;
    const int c = (int)((id / HW) % C);
    const float inv = 1.0f / sqrtf(var[c] + eps);
    float v = (x[id] - mean[c]) * inv;
    if (gamma) v = v * gamma[c];
    if (beta) v = v + beta[c];
    y[id] = v;
}

bool conv_geometry(int64_t H, int64_t W, int KH, int KW, int sh, int sw, int pt, int pb, int pl, int pr,
                   int dh, int dw, int64_t* OH, int64_t* OW) {
    if (KH < 1 || KW < 1 || sh < 1 || sw < 1 || dh < 1 || dw < 1 || pt < 0 || pb < 0 || pl < 0 || pr < 0)
        return false;
    const int64_t eh = (int64_t)dh * (KH - 1) + 1, ew = (int64_t)dw * (KW - 1) + 1;
    const int64_t hp = H + pt + pb, wp = W + pl + pr;
    if (hp < eh || wp < ew) return false;
    *OH = (hp - eh) / sh + 1;
    *OW = (wp - ew) / sw + 1;
    return true;
}

constexpr int64_t CV_MAX = (int64_t)1 << 31;

// Packed weight row stride: K rounded up to whole 128-byte stages.
int64_t conv_ldw(int64_t K) { return (K + 127) / 128 * 128; }

// Launch plan of lq_conv2d_i8, shared by the call and its workspace query.
struct ConvPlan {
    bool dma, big;
    bool taps;      // tap-im2col form: packed input [n][hp][ow][g][32], a KH x 1 convolution
    int64_t Cp, ldw, gx, gy;
    int splits;
    size_t pack_bytes;  // padded NHWC input (rounded up to 256 bytes)
    size_t part_bytes;  // split-K tile sums
};

ConvPlan conv_plan(int64_t N, int64_t C, int64_t H, int64_t W, int64_t Cout, int64_t KH, int64_t KW, int pt, int pb,
                   int pl, int pr, int64_t OH, int64_t OW, int64_t groups) {
    ConvPlan p{};
    const int64_t Cg = C / groups, Cout_g = Cout / groups;
    p.taps = conv_taps_form(Cg, KW);
    p.Cp = p.taps ? CV_TAPS_CP : (Cg + 15) / 16 * 16;
    const int64_t Wpk = p.taps ? OW : W + pl + pr;  // packed input width
    p.pack_bytes = (size_t)((N * (H + pt + pb) * Wpk * groups * p.Cp + 255) / 256 * 256);
    const int64_t K = KH * (p.taps ? 1 : KW) * p.Cp;
    p.ldw = conv_ldw(K);
    const int64_t ntaps = (p.ldw + p.Cp - 1) / p.Cp;
    const bool pow2 = p.Cp <= 128 && (p.Cp & (p.Cp - 1)) == 0;
    const int64_t P = N * OH * OW;
    p.dma = (pow2 || p.Cp % 128 == 0) && ntaps <= CV_MAX_TAPS && Cout_g * p.ldw < CV_MAX;
    p.splits = 1;
    if (!p.dma) return p;
    p.gy = (Cout_g + 63) / 64;
    p.big = ((P + 255) / 256) * p.gy * groups >= 256;
    p.gx = (P + (p.big ? 255 : 127)) / (p.big ? 256 : 128);
    // fewer tiles than CUs and a long K: split K so every CU has a tile (at least four
    // 128-byte stages per split)
    const int64_t tiles = p.gx * p.gy * groups;
    const int64_t nk = p.ldw / 128;
    // (below 128 tiles: at 196 tiles a 2-way split measured slower than none)
    if (!p.big && tiles < 128 && nk >= 8) {
        int64_t sp = std::min<int64_t>((256 + tiles - 1) / tiles, nk / 4);
        while (sp > 1 && (sp - 1) * ((nk + sp - 1) / sp) >= nk) --sp;
        if (sp > 1 && tiles * sp <= 65535) {
            p.splits = (int)sp;
            p.part_bytes = (size_t)(tiles * sp * 128 * 64 * 4);
        }
    }
    return p;
}

}  // namespace
}  // namespace lq

using namespace lq;

extern "C" {

size_t lq_conv2d_weight_pack_size(int64_t Cout, int64_t Cin_g, int64_t KH, int64_t KW) {
    if (Cout < 0 || Cin_g < 1 || KH < 1 || KW < 1) return 0;
    if (conv_taps_form(Cin_g, KW)) return (size_t)(Cout * conv_ldw(KH * CV_TAPS_CP));
    const int64_t Cp = (Cin_g + 15) / 16 * 16;
    return (size_t)(Cout * conv_ldw(KH * KW * Cp));
}

int lq_conv2d_pack_weights_i8(const int8_t* d_w, int64_t Cout, int64_t Cin_g, int64_t KH, int64_t KW,
                              int8_t* d_w_packed, int32_t* d_w_sums, void* stream) {
    LQ_REQUIRE(Cout >= 0 && Cin_g >= 1 && KH >= 1 && KW >= 1 && Cout * Cin_g * KH * KW < CV_MAX,
               "lq_conv2d_pack_weights_i8: bad shape");
    if (Cout == 0) return LQ_OK;
    LQ_REQUIRE(d_w && d_w_packed, "lq_conv2d_pack_weights_i8: NULL pointer");
    const int Cp = (int)((Cin_g + 15) / 16 * 16);
    hipStream_t st = as_stream(stream);
    if (conv_taps_form(Cin_g, KW)) {
        const int64_t ldw = conv_ldw(KH * CV_TAPS_CP);
        const int64_t chunks = Cout * (ldw / 16);
        hipLaunchKernelGGL(conv_pack_weights_taps_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, st,
                           d_w, (int)Cout, (int)Cin_g, (int)KH, (int)KW, (int)ldw, d_w_packed);
    } else {
        const int64_t ldw = conv_ldw(KH * KW * Cp);
        const int64_t chunks = Cout * (ldw / 16);
        hipLaunchKernelGGL(conv_pack_weights_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, st, d_w,
                           (int)Cout, (int)Cin_g, (int)KH, (int)KW, Cp, (int)ldw, d_w_packed);
    }
    if (d_w_sums)
        hipLaunchKernelGGL(conv_weight_sums_kernel, dim3((unsigned)((Cout + 3) / 4)), dim3(256), 0, st, d_w, (int)Cout,
                           Cin_g * KH * KW, d_w_sums);
    return launch_status("lq_conv2d_pack_weights_i8");
}

size_t lq_conv2d_i8_workspace_size(int64_t N, int64_t C, int64_t H, int64_t W, int64_t Cout, int64_t KH, int64_t KW,
                                   int stride_h, int stride_w, int pad_top, int pad_bottom, int pad_left,
                                   int pad_right, int dilation_h, int dilation_w, int64_t groups) {
    if (N < 0 || C < 1 || H < 1 || W < 1 || Cout < 1 || groups < 1 || C % groups || Cout % groups) return 0;
    int64_t OH = 0, OW = 0;
    if (!conv_geometry(H, W, (int)KH, (int)KW, stride_h, stride_w, pad_top, pad_bottom, pad_left, pad_right,
                       dilation_h, dilation_w, &OH, &OW))
        return 0;
    const ConvPlan pl = conv_plan(N, C, H, W, Cout, KH, KW, pad_top, pad_bottom, pad_left, pad_right, OH, OW, groups);
    return pl.pack_bytes + pl.part_bytes;
}

int lq_conv2d_i8(const int8_t* d_x, int x_code_type, int64_t N, int64_t C, int64_t H, int64_t W,
                 const int8_t* d_w_packed, const int32_t* d_w_sums, int64_t Cout, int64_t KH, int64_t KW,
                 int stride_h, int stride_w, int pad_top, int pad_bottom, int pad_left, int pad_right,
                 int dilation_h, int dilation_w, int64_t groups, int padding_mode, const float* d_a_scale,
                 const float* d_a_zero_point, const float* d_w_scale, const float* d_bias,
                 const float* d_out_scale, const float* d_out_zero_point, int out_qmin, int out_qmax,
                 int out_kind, int flags, void* d_y, void* d_workspace, size_t workspace_bytes, void* stream) {
    LQ_REQUIRE(N >= 0 && C >= 1 && H >= 1 && W >= 1 && Cout >= 1 && groups >= 1,
               "lq_conv2d_i8: bad shape");
    LQ_REQUIRE(C % groups == 0 && Cout % groups == 0, "lq_conv2d_i8: channels must divide by groups");
    LQ_REQUIRE(x_code_type == LQ_I8 || x_code_type == LQ_U8S8, "lq_conv2d_i8: activation codes must be LQ_I8 or LQ_U8S8");
    LQ_REQUIRE(padding_mode >= LQ_PAD_ZEROS && padding_mode <= LQ_PAD_CIRCULAR, "lq_conv2d_i8: unknown padding mode");
    LQ_REQUIRE((flags & ~(LQ_EPI_RELU | LQ_CONV_OUT_NHWC)) == 0, "lq_conv2d_i8: unknown flags");
    const bool out_nhwc = (flags & LQ_CONV_OUT_NHWC) != 0;
    LQ_REQUIRE(!out_nhwc || ((out_kind == LQ_OUT_Q8 || out_kind == LQ_OUT_QU8 || out_kind == LQ_OUT_QU8S8) &&
                             groups == 1 && Cout % 16 == 0 && aligned16(d_y)),
               "lq_conv2d_i8: LQ_CONV_OUT_NHWC needs byte codes out, groups 1, Cout a multiple of 16 and a "
               "16-byte aligned output");
    LQ_REQUIRE(out_kind >= LQ_OUT_I32 && out_kind <= LQ_OUT_QU8S8, "lq_conv2d_i8: unknown out_kind");
    int64_t OH = 0, OW = 0;
    LQ_REQUIRE(conv_geometry(H, W, (int)KH, (int)KW, stride_h, stride_w, pad_top, pad_bottom, pad_left, pad_right,
                             dilation_h, dilation_w, &OH, &OW),
               "lq_conv2d_i8: kernel, stride, padding or dilation do not fit the input");
    if (padding_mode != LQ_PAD_ZEROS)
        LQ_REQUIRE(pad_top < H && pad_bottom < H && pad_left < W && pad_right < W,
                   "lq_conv2d_i8: reflect / replicate / circular padding must be smaller than the input");
    if (N == 0) return LQ_OK;
    const int64_t Cg = C / groups, Cout_g = Cout / groups;
    // the packed input's geometry: padded NHWC, or the tap-im2col form (a KH x 1 convolution
    // at horizontal stride 1 over 32 bytes per position, the packing applied the columns)
    const bool taps = conv_taps_form(Cg, KW);
    const int64_t Cp = taps ? CV_TAPS_CP : (Cg + 15) / 16 * 16;
    const int64_t Hp = H + pad_top + pad_bottom, Wp = taps ? OW : W + pad_left + pad_right;
    const int64_t KWe = taps ? 1 : KW;
    const int swe = taps ? 1 : stride_w, dwe = taps ? 1 : dilation_w;
    const int64_t P = N * OH * OW;
    const int64_t K = KH * KWe * Cp;
    LQ_REQUIRE(N * C * H * W < CV_MAX && N * Hp * Wp * groups * Cp < CV_MAX && P < CV_MAX && N * Cout * OH * OW < CV_MAX,
               "lq_conv2d_i8: tensors above 2^31 elements are not supported");
    LQ_REQUIRE(d_x && d_w_packed && d_w_scale && d_y, "lq_conv2d_i8: NULL pointer");
    const bool has_za = d_a_zero_point != nullptr || x_code_type == LQ_U8S8;
    LQ_REQUIRE(!has_za || d_w_sums, "lq_conv2d_i8: an activation zero point needs the weight sums d_w_sums");
    LQ_REQUIRE(aligned16(d_w_packed) && aligned16(d_workspace), "lq_conv2d_i8: packed weights and workspace must be 16-byte aligned");
    const ConvPlan plan = conv_plan(N, C, H, W, Cout, KH, KW, pad_top, pad_bottom, pad_left, pad_right, OH, OW, groups);
    LQ_REQUIRE(d_workspace && workspace_bytes >= plan.pack_bytes + plan.part_bytes,
               "lq_conv2d_i8: workspace smaller than lq_conv2d_i8_workspace_size");
    if (out_nhwc && !plan.dma)
        return set_error(LQ_ERR_UNSUPPORTED, "lq_conv2d_i8: LQ_CONV_OUT_NHWC needs the LDS-DMA plan");
    hipStream_t st = as_stream(stream);

    // halo-staged direct kernel: no padded copy of the input (the workspace goes unused)
    // (integer-code outputs only: the float kinds' epilogue does not fit this kernel's
    // register budget without spilling)
    const bool halo_kind = out_kind == LQ_OUT_Q8 || out_kind == LQ_OUT_QU8 || out_kind == LQ_OUT_QU8S8;
    const int64_t halo = (halo_kind && !out_nhwc && (reinterpret_cast<uintptr_t>(d_x) & 15) == 0 && !plan.taps &&
                          plan.Cp == C)
                             ? halo_bytes_for(N, C, H, W, Cout, KH, KW, stride_h, stride_w, pad_top, pad_bottom,
                                              pad_left, pad_right, dilation_h, dilation_w, groups, padding_mode, OH, OW)
                             : 0;
    if (halo > 0) {
        HaloArgs hg{};
        ConvDmaArgs& d = hg.e;
        d.wp = d_w_packed;
        d.y = d_y;
        d.G = 1; d.Cp = (int)C; d.Cout_g = (int)Cout; d.KH = (int)KH; d.KW = (int)KW; d.sh = 1; d.sw = 1;
        d.dh = 1; d.dw = 1; d.OH = (int)OH; d.OW = (int)OW; d.P = (int)P; d.ldw = (int)plan.ldw;
        d.a_scale = d_a_scale; d.a_zp = d_a_zero_point; d.a_u8s8 = x_code_type == LQ_U8S8;
        d.w_scale = d_w_scale; d.w_sums = d_w_sums; d.bias = d_bias;
        d.out_scale = d_out_scale; d.out_zp = d_out_zero_point;
        d.qmin = out_qmin; d.qmax = out_qmax; d.relu = (flags & LQ_EPI_RELU) ? 1 : 0;
        d.splits = 1; d.phase = 1;
        hg.x = d_x;
        hg.N = (int)N; hg.C = (int)C; hg.H = (int)H; hg.W = (int)W;
        hg.Hp = (int)(H + pad_top + pad_bottom); hg.Wp = (int)(W + pad_left + pad_right);
        hg.pt = pad_top; hg.pl = pad_left; hg.KH = (int)KH; hg.KW = (int)KW; hg.nc = (int)(C / 64);
        hg.halo_bytes = (int)halo;
        hg.inv_ohw = 1.0f / (float)(OH * OW);
        hg.inv_ow = 1.0f / (float)OW;
        hg.inv_hp = 1.0f / (float)hg.Hp;
        hg.inv_w = 1.0f / (float)W;
        hg.dummy_pos = (int)((halo - 1024) / 64);
        const size_t lds = (size_t)halo + (size_t)(KH * KW) * 4096;
        const dim3 grid((unsigned)((P + 255) / 256), (unsigned)(Cout / 64));
#define LQ_CONV_HALO(K_)                                                                                    \
    {                                                                                                       \
        const hipError_t e_ = hipFuncSetAttribute(reinterpret_cast<const void*>(&conv_i8_halo_kernel<K_>),  \
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);     \
        if (e_ != hipSuccess) return set_error(LQ_ERR_HIP, std::string("lq_conv2d_i8 (halo): ") + hipGetErrorString(e_)); \
        hipLaunchKernelGGL((conv_i8_halo_kernel<K_>), grid, dim3(256), lds, st, hg);                        \
    }                                                                                                       \
    break;
        switch (out_kind) {
            case LQ_OUT_Q8: LQ_CONV_HALO(LQ_OUT_Q8)
            case LQ_OUT_QU8: LQ_CONV_HALO(LQ_OUT_QU8)
            default: LQ_CONV_HALO(LQ_OUT_QU8S8)
        }
#undef LQ_CONV_HALO
        note_path("conv halo");
        return launch_status("lq_conv2d_i8");
    }

    PackArgs pa{};
    pa.x = d_x;
    pa.xp = static_cast<int8_t*>(d_workspace);
    pa.N = (int)N; pa.C = (int)C; pa.H = (int)H; pa.W = (int)W; pa.G = (int)groups; pa.Cg = (int)Cg;
    pa.Cp = (int)Cp; pa.Hp = (int)Hp; pa.Wp = (int)Wp; pa.pt = pad_top; pa.pl = pad_left;
    pa.mode = padding_mode;
    pa.a_zp = d_a_zero_point;
    pa.a_u8s8 = x_code_type == LQ_U8S8;
    LQ_REQUIRE(N * groups <= 65535, "lq_conv2d_i8: N * groups must be <= 65535");
    PackGeom pg{};
    pg.pb = pad_bottom;
    pg.pr = pad_right;
    pg.all_cells = H * W < 128;  // a plane under half a tile: gather every position
    pg.ptiles = pg.all_cells ? 0 : (int)((H * W + 255) / 256);
    pg.tiles = pg.ptiles * (int)((Cp + CV_PCB - 1) / CV_PCB);
    pg.border_cells = pg.all_cells ? (int)(Hp * Wp) : (int)((pad_top + pad_bottom) * Wp + H * (pad_left + pad_right));
    const int bblocks = (int)((pg.border_cells * (Cp / 16) + 255) / 256);
    const dim3 pgrid((unsigned)(pg.tiles + bblocks), (unsigned)(N * groups));
    if (taps) {
        TapsArgs ta{};
        ta.x = d_x;
        ta.xp = pa.xp;
        ta.N = (int)N; ta.C = (int)C; ta.H = (int)H; ta.W = (int)W; ta.G = (int)groups; ta.Cg = (int)Cg;
        ta.Hp = (int)Hp; ta.OW = (int)OW; ta.KW = (int)KW; ta.sw = stride_w; ta.dw = dilation_w;
        ta.pt = pad_top; ta.pl = pad_left; ta.mode = padding_mode;
        ta.a_zp = d_a_zero_point; ta.a_u8s8 = pa.a_u8s8;
        // output columns per workgroup: as many of CV_TAPS_OWB as the staged rows hold
        const int64_t reach = (KW - 1) * (int64_t)dilation_w + 1;
        LQ_REQUIRE(reach <= CV_TAPS_SPAN, "lq_conv2d_i8: dilated kernel row wider than the tap staging buffer");
        ta.owb = (int)std::min<int64_t>(CV_TAPS_OWB, (CV_TAPS_SPAN - reach) / stride_w + 1);
        ta.span = (int)((ta.owb - 1) * (int64_t)stride_w + reach);
        const int64_t hblocks = (Hp + CV_TAPS_ROWS - 1) / CV_TAPS_ROWS;
        LQ_REQUIRE(N * hblocks <= 2147483647LL && (OW + ta.owb - 1) / ta.owb <= 65535,
                   "lq_conv2d_i8: too many input rows or output columns for the tap packing");
        const dim3 tgrid((unsigned)(N * hblocks), (unsigned)((OW + ta.owb - 1) / ta.owb));
        hipLaunchKernelGGL(conv_pack_taps_kernel, tgrid, dim3(256), 0, st, ta);
    } else if ((H * W) % 4 == 0 && (reinterpret_cast<uintptr_t>(d_x) & 3) == 0) {
        hipLaunchKernelGGL(conv_pack_input_kernel<true>, pgrid, dim3(256), 0, st, pa, pg);
    } else {
        hipLaunchKernelGGL(conv_pack_input_kernel<false>, pgrid, dim3(256), 0, st, pa, pg);
    }

    ConvArgs a{};
    a.xp = pa.xp;
    a.wp = d_w_packed;
    a.y = d_y;
    a.N = (int)N; a.Hp = (int)Hp; a.Wp = (int)Wp; a.G = (int)groups; a.Cp = (int)Cp; a.Cout_g = (int)Cout_g;
    a.KH = (int)KH; a.KW = (int)KWe; a.sh = stride_h; a.sw = swe; a.dh = dilation_h; a.dw = dwe;
    a.OH = (int)OH; a.OW = (int)OW; a.K = (int)K; a.P = (int)P; a.ldw = (int)conv_ldw(K);
    a.a_scale = d_a_scale;
    a.a_zp = d_a_zero_point;
    a.a_u8s8 = pa.a_u8s8;
    a.w_scale = d_w_scale;
    a.w_sums = d_w_sums;
    a.bias = d_bias;
    a.out_scale = d_out_scale;
    a.out_zp = d_out_zero_point;
    a.qmin = out_qmin;
    a.qmax = out_qmax;
    a.relu = (flags & LQ_EPI_RELU) ? 1 : 0;
    // LDS-DMA kernel: whole 16-byte chunks of one tap per copy (Cp a power of two up to 128,
    // or a multiple of 128) and a tap table that fits.
    const int64_t ldw = plan.ldw;
    const bool pow2 = Cp <= 128 && (Cp & (Cp - 1)) == 0;
    if (plan.dma) {
        ConvDmaArgs d{};
        d.xp = pa.xp;
        d.wp = d_w_packed;
        d.y = d_y;
        d.xp_bytes = (uint32_t)(N * Hp * Wp * groups * Cp);
        d.Hp = (int)Hp; d.Wp = (int)Wp; d.G = (int)groups; d.Cp = (int)Cp;
        d.cp_shift = pow2 ? __builtin_ctz((unsigned)Cp) : -1;
        d.Cout_g = (int)Cout_g; d.KH = (int)KH; d.KW = (int)KWe; d.sh = stride_h; d.sw = swe;
        d.dh = dilation_h; d.dw = dwe; d.OH = (int)OH; d.OW = (int)OW; d.P = (int)P;
        d.nk = (int)(ldw / 128); d.ldw = (int)ldw;
        d.kw_magic = (int)((65536 + KWe - 1) / KWe);
        d.kh_stride = (int)(dilation_h * Wp * groups * Cp);
        d.kw_stride = (int)(dwe * groups * Cp);
        d.a_scale = d_a_scale; d.a_zp = d_a_zero_point; d.a_u8s8 = pa.a_u8s8;
        d.w_scale = d_w_scale; d.w_sums = d_w_sums; d.bias = d_bias;
        d.out_scale = d_out_scale; d.out_zp = d_out_zero_point;
        d.qmin = out_qmin; d.qmax = out_qmax; d.relu = a.relu;
        d.splits = plan.splits;
        d.part = reinterpret_cast<int32_t*>(static_cast<int8_t*>(d_workspace) + plan.pack_bytes);
        if (out_nhwc) {
            d.out_nhwc = 1;
            d.ypad = 0;
            d.ycs = (int)Cout;
            d.yrow = OW * Cout;
            d.yimg = OH * OW * Cout;
        }
        const bool big = plan.big;
        const dim3 grid((unsigned)plan.gx, (unsigned)plan.gy, (unsigned)groups);
        const dim3 grid0((unsigned)plan.gx, (unsigned)plan.gy, (unsigned)(groups * plan.splits));
        ConvDmaArgs d1 = d;
        d.phase = 0;
        d1.phase = 1;
#define LQ_CONV_DMA(K_)                                                                                        \
    if (big) {                                                                                                 \
        hipLaunchKernelGGL((conv_i8_dma_kernel<256, 64, 4, 1, 2, K_>), grid, dim3(256), 0, st, d);            \
    } else {                                                                                                   \
        hipLaunchKernelGGL((conv_i8_dma_kernel<128, 64, 2, 2, CV_SMALL_NBUF, K_>), grid0, dim3(256), 0, st, d); \
        if (plan.splits > 1)                                                                                   \
            hipLaunchKernelGGL((conv_i8_dma_kernel<128, 64, 2, 2, CV_SMALL_NBUF, K_>), grid, dim3(256), 0, st, d1); \
    }                                                                                                          \
    break;
#define LQ_CONV_DMA_NHWC(K_)                                                                                   \
    if (big) {                                                                                                 \
        hipLaunchKernelGGL((conv_i8_dma_kernel<256, 64, 4, 1, 2, K_, true>), grid, dim3(256), 0, st, d);      \
    } else {                                                                                                   \
        hipLaunchKernelGGL((conv_i8_dma_kernel<128, 64, 2, 2, CV_SMALL_NBUF, K_, true>), grid0, dim3(256), 0, st, d); \
        if (plan.splits > 1)                                                                                   \
            hipLaunchKernelGGL((conv_i8_dma_kernel<128, 64, 2, 2, CV_SMALL_NBUF, K_, true>), grid, dim3(256), 0, st, d1); \
    }                                                                                                          \
    break;
        if (out_nhwc) {
            switch (out_kind) {
                case LQ_OUT_Q8: LQ_CONV_DMA_NHWC(LQ_OUT_Q8)
                case LQ_OUT_QU8: LQ_CONV_DMA_NHWC(LQ_OUT_QU8)
                default: LQ_CONV_DMA_NHWC(LQ_OUT_QU8S8)
            }
            note_path(plan.taps ? "conv taps dma nhwc out" : "conv dma nhwc out");
            return launch_status("lq_conv2d_i8");
        }
#undef LQ_CONV_DMA_NHWC
        switch (out_kind) {
            case LQ_OUT_I32: LQ_CONV_DMA(LQ_OUT_I32)
            case LQ_OUT_F32: LQ_CONV_DMA(LQ_OUT_F32)
            case LQ_OUT_F16: LQ_CONV_DMA(LQ_OUT_F16)
            case LQ_OUT_Q8: LQ_CONV_DMA(LQ_OUT_Q8)
            case LQ_OUT_QU8: LQ_CONV_DMA(LQ_OUT_QU8)
            case LQ_OUT_FQ32: LQ_CONV_DMA(LQ_OUT_FQ32)
            case LQ_OUT_Q16: LQ_CONV_DMA(LQ_OUT_Q16)
            default: LQ_CONV_DMA(LQ_OUT_QU8S8)
        }
#undef LQ_CONV_DMA
        if (taps)
            note_path(big ? "conv taps dma 256x64" : plan.splits > 1 ? "conv taps dma 128x64 split-k" : "conv taps dma 128x64");
        else
            note_path(big ? "conv dma 256x64" : plan.splits > 1 ? "conv dma 128x64 split-k" : "conv dma 128x64");
        return launch_status("lq_conv2d_i8");
    }
    const dim3 grid((unsigned)((P + CV_BM - 1) / CV_BM), (unsigned)((Cout_g + CV_BN - 1) / CV_BN), (unsigned)groups);
    switch (out_kind) {
        case LQ_OUT_I32: hipLaunchKernelGGL(conv_i8_kernel<LQ_OUT_I32>, grid, dim3(CV_THREADS), 0, st, a); break;
        case LQ_OUT_F32: hipLaunchKernelGGL(conv_i8_kernel<LQ_OUT_F32>, grid, dim3(CV_THREADS), 0, st, a); break;
        case LQ_OUT_F16: hipLaunchKernelGGL(conv_i8_kernel<LQ_OUT_F16>, grid, dim3(CV_THREADS), 0, st, a); break;
        case LQ_OUT_Q8: hipLaunchKernelGGL(conv_i8_kernel<LQ_OUT_Q8>, grid, dim3(CV_THREADS), 0, st, a); break;
        case LQ_OUT_QU8: hipLaunchKernelGGL(conv_i8_kernel<LQ_OUT_QU8>, grid, dim3(CV_THREADS), 0, st, a); break;
        case LQ_OUT_FQ32: hipLaunchKernelGGL(conv_i8_kernel<LQ_OUT_FQ32>, grid, dim3(CV_THREADS), 0, st, a); break;
        case LQ_OUT_Q16: hipLaunchKernelGGL(conv_i8_kernel<LQ_OUT_Q16>, grid, dim3(CV_THREADS), 0, st, a); break;
        default: hipLaunchKernelGGL(conv_i8_kernel<LQ_OUT_QU8S8>, grid, dim3(CV_THREADS), 0, st, a); break;
    }
    note_path(taps ? "conv taps staged 128x64" : "conv staged 128x64");
    return launch_status("lq_conv2d_i8");
}

size_t lq_conv2d_i8_nhwc_workspace_size(int64_t N, int64_t C, int64_t H, int64_t W, int64_t Cout, int64_t KH,
                                        int64_t KW, int stride, int pad) {
    if (N < 0 || C < 1 || H < 1 || W < 1 || Cout < 1) return 0;
    int64_t OH = 0, OW = 0;
    if (!conv_geometry(H, W, (int)KH, (int)KW, stride, stride, pad, pad, pad, pad, 1, 1, &OH, &OW)) return 0;
    const ConvPlan pl = conv_plan(N, C, H, W, Cout, KH, KW, pad, pad, pad, pad, OH, OW, 1);
    return pl.part_bytes;
}

int lq_conv2d_i8_nhwc(const int8_t* d_x, int x_code_type, int64_t N, int64_t C, int64_t H, int64_t W, int x_pad,
                      int64_t x_cs, const int8_t* d_w_packed, const int32_t* d_w_sums, int64_t Cout, int64_t KH,
                      int64_t KW, int stride, int pad, const float* d_a_scale, const float* d_a_zero_point,
                      const float* d_w_scale, const float* d_bias, const float* d_out_scale,
                      const float* d_out_zero_point, int out_qmin, int out_qmax, int out_kind, int flags, int8_t* d_y,
                      int y_pad, int64_t y_cs, const int8_t* d_skip, int skip_type, const float* d_skip_scale,
                      const float* d_skip_zero_point, const float* d_merge_scale, const float* d_merge_zero_point,
                      int merge_qmin, int merge_qmax, int merge_type, int merge_flags, void* d_workspace,
                      size_t workspace_bytes, void* stream) {
    const char* fn = "lq_conv2d_i8_nhwc";
    LQ_REQUIRE(N >= 0 && C >= 1 && H >= 1 && W >= 1 && Cout >= 1 && KH >= 1 && KW >= 1 && stride >= 1 && pad >= 0,
               std::string(fn) + ": bad shape");
    LQ_REQUIRE(x_code_type == LQ_I8 || x_code_type == LQ_U8S8, std::string(fn) + ": activation codes must be LQ_I8 or LQ_U8S8");
    LQ_REQUIRE(out_kind == LQ_OUT_Q8 || out_kind == LQ_OUT_QU8 || out_kind == LQ_OUT_QU8S8,
               std::string(fn) + ": byte codes out (LQ_OUT_Q8 / QU8 / QU8S8)");
    LQ_REQUIRE((flags & ~LQ_EPI_RELU) == 0 && (merge_flags & ~LQ_EPI_RELU) == 0, std::string(fn) + ": unknown flags");
    LQ_REQUIRE(x_pad >= pad && y_pad >= 0 && y_pad <= 1, std::string(fn) + ": the input border must cover the padding; "
                                                                            "an output border of 0 or 1");
    LQ_REQUIRE(x_cs >= C && x_cs % 16 == 0 && y_cs >= Cout && Cout % 16 == 0,
               std::string(fn) + ": channel strides: x_cs >= C, a multiple of 16; y_cs >= Cout; Cout a multiple of 16");
    LQ_REQUIRE(!d_skip || ((skip_type == LQ_I8 || skip_type == LQ_U8 || skip_type == LQ_U8S8) &&
                           (merge_type == LQ_I8 || merge_type == LQ_U8 || merge_type == LQ_U8S8) && d_skip_scale &&
                           d_merge_scale),
               std::string(fn) + ": a skip needs byte code types and its and the merge's scales");
    int64_t OH = 0, OW = 0;
    LQ_REQUIRE(conv_geometry(H, W, (int)KH, (int)KW, stride, stride, pad, pad, pad, pad, 1, 1, &OH, &OW),
               std::string(fn) + ": kernel, stride or padding do not fit the input");
    if (N == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_w_packed && d_w_scale && d_y, std::string(fn) + ": NULL pointer");
    const bool has_za = d_a_zero_point != nullptr || x_code_type == LQ_U8S8;
    LQ_REQUIRE(!has_za || d_w_sums, std::string(fn) + ": an activation zero point needs the weight sums d_w_sums");
    const int64_t Cp = (C + 15) / 16 * 16;
    LQ_REQUIRE(!conv_taps_form(C, KW) && x_cs == Cp, std::string(fn) + ": the input's channel stride must be C rounded "
                                                                       "up to 16 (and C above the tap-im2col form)");
    const ConvPlan plan = conv_plan(N, C, H, W, Cout, KH, KW, pad, pad, pad, pad, OH, OW, 1);
    if (!plan.dma) return set_error(LQ_ERR_UNSUPPORTED, std::string(fn) + ": this geometry has no LDS-DMA plan");
    LQ_REQUIRE(plan.part_bytes == 0 || (d_workspace && aligned16(d_workspace) && workspace_bytes >= plan.part_bytes),
               std::string(fn) + ": workspace smaller than lq_conv2d_i8_nhwc_workspace_size");
    LQ_REQUIRE(aligned16(d_w_packed) && aligned16(d_x) && aligned16(d_y) && (!d_skip || aligned16(d_skip)) &&
                   y_cs % 16 == 0,
               std::string(fn) + ": 16-byte aligned buffers and an output channel stride that is a multiple of 16");
    // the input buffer's geometry, and the origin the convolution's own padding starts at
    const int64_t Hpb = H + 2 * x_pad, Wpb = W + 2 * x_pad;
    const int64_t shift = x_pad - pad;
    const int8_t* xo = d_x + (shift * Wpb + shift) * Cp;
    const int64_t xbytes = N * Hpb * Wpb * Cp - (shift * Wpb + shift) * Cp;
    const int64_t P = N * OH * OW;
    LQ_REQUIRE(N * Hpb * Wpb * Cp < CV_MAX && P < CV_MAX && N * (OH + 2 * y_pad) * (OW + 2 * y_pad) * y_cs < CV_MAX,
               std::string(fn) + ": tensors above 2^31 bytes are not supported");
    const hipStream_t st = as_stream(stream);
    ConvDmaArgs d{};
    d.xp = xo;
    d.wp = d_w_packed;
    d.y = d_y;  // the padded buffer's first byte: the epilogue adds the border offsets
    d.xp_bytes = (uint32_t)xbytes;
    d.Hp = (int)Hpb; d.Wp = (int)Wpb; d.G = 1; d.Cp = (int)Cp;
    const bool pow2 = Cp <= 128 && (Cp & (Cp - 1)) == 0;
    d.cp_shift = pow2 ? __builtin_ctz((unsigned)Cp) : -1;
    d.Cout_g = (int)Cout; d.KH = (int)KH; d.KW = (int)KW; d.sh = stride; d.sw = stride;
    d.dh = 1; d.dw = 1; d.OH = (int)OH; d.OW = (int)OW; d.P = (int)P;
    d.nk = (int)(plan.ldw / 128); d.ldw = (int)plan.ldw;
    d.kw_magic = (int)((65536 + KW - 1) / KW);
    d.kh_stride = (int)(Wpb * Cp);
    d.kw_stride = (int)Cp;
    d.a_scale = d_a_scale; d.a_zp = d_a_zero_point; d.a_u8s8 = x_code_type == LQ_U8S8;
    d.w_scale = d_w_scale; d.w_sums = d_w_sums; d.bias = d_bias;
    d.out_scale = d_out_scale; d.out_zp = d_out_zero_point;
    d.qmin = out_qmin; d.qmax = out_qmax; d.relu = (flags & LQ_EPI_RELU) ? 1 : 0;
    d.splits = plan.splits;
    d.part = static_cast<int32_t*>(d_workspace);
    d.out_nhwc = 1;
    d.ypad = y_pad;
    d.ycs = (int)y_cs;
    d.yrow = (OW + 2 * y_pad) * y_cs;
    d.yimg = (OH + 2 * y_pad) * d.yrow;
    d.skip = d_skip;
    d.skip_type = skip_type;
    d.skip_scale = d_skip_scale;
    d.skip_zp = d_skip_zero_point;
    d.m_scale = d_merge_scale;
    d.m_zp = d_merge_zero_point;
    d.m_qmin = merge_qmin;
    d.m_qmax = merge_qmax;
    d.m_type = merge_type;
    d.m_relu = (merge_flags & LQ_EPI_RELU) ? 1 : 0;
    // At most 256 tiles of 128 x 64 (at most one per CU): the tile's K stages split between
    // two or three wave groups of one workgroup (their sums meet in LDS) in place of the
    // cross-workgroup split and its second launch.  At most 128 such tiles and three groups:
    // 64 x 64 tiles with three-stage rings (twice the workgroups, a deeper prefetch; the
    // 144 KiB of LDS still fit one workgroup per CU).
    const int64_t tiles = plan.gx * plan.gy;
    const int ksplit = plan.big || tiles > 256 || d.nk < 6 ? 1 : d.nk % 3 == 0 ? 3 : d.nk % 2 == 0 ? 2 : 1;
    const bool t64 = ksplit == 3 && tiles <= 128;
    if (ksplit > 1) d.splits = 1;
    const int splits = d.splits;
    const dim3 grid((unsigned)plan.gx, (unsigned)plan.gy, 1u);
    const dim3 grid0((unsigned)plan.gx, (unsigned)plan.gy, (unsigned)splits);
    const dim3 grid64((unsigned)((P + 63) / 64), (unsigned)plan.gy, 1u);
    ConvDmaArgs d1 = d;
    d.phase = 0;
    d1.phase = 1;
#define LQ_CONV_NHWC(K_)                                                                                        \
    if (plan.big) {                                                                                              \
        hipLaunchKernelGGL((conv_i8_dma_kernel<256, 64, 4, 1, 2, K_, true>), grid, dim3(256), 0, st, d);        \
    } else if (t64) {                                                                                            \
        hipLaunchKernelGGL((conv_i8_dma_kernel<64, 64, 1, 2, 3, K_, true, 3>), grid64, dim3(384), 0, st, d);    \
    } else if (ksplit == 3) {                                                                                    \
        hipLaunchKernelGGL((conv_i8_dma_kernel<128, 64, 2, 2, CV_SMALL_NBUF, K_, true, 3>), grid, dim3(768), 0, st, d); \
    } else if (ksplit == 2) {                                                                                    \
        hipLaunchKernelGGL((conv_i8_dma_kernel<128, 64, 2, 2, CV_SMALL_NBUF, K_, true, 2>), grid, dim3(512), 0, st, d); \
    } else {                                                                                                     \
        hipLaunchKernelGGL((conv_i8_dma_kernel<128, 64, 2, 2, CV_SMALL_NBUF, K_, true>), grid0, dim3(256), 0, st, d); \
        if (splits > 1)                                                                                          \
            hipLaunchKernelGGL((conv_i8_dma_kernel<128, 64, 2, 2, CV_SMALL_NBUF, K_, true>), grid, dim3(256), 0, st, d1); \
    }                                                                                                            \
    break;
    switch (out_kind) {
        case LQ_OUT_Q8: LQ_CONV_NHWC(LQ_OUT_Q8)
        case LQ_OUT_QU8: LQ_CONV_NHWC(LQ_OUT_QU8)
        default: LQ_CONV_NHWC(LQ_OUT_QU8S8)
    }
#undef LQ_CONV_NHWC
    note_path(plan.big ? "conv nhwc dma 256x64"
              : t64        ? "conv nhwc dma 64x64 wave-group split-k"
              : ksplit > 1 ? "conv nhwc dma 128x64 wave-group split-k"
              : splits > 1 ? "conv nhwc dma 128x64 split-k"
                           : "conv nhwc dma 128x64");
    return launch_status(fn);
}

int lq_conv2d_f32(const float* d_x, int64_t N, int64_t C, int64_t H, int64_t W, const float* d_w,
                  const float* d_bias, int64_t Cout, int64_t KH, int64_t KW, int stride_h, int stride_w,
                  int pad_top, int pad_bottom, int pad_left, int pad_right, int dilation_h, int dilation_w,
                  int64_t groups, int padding_mode, float* d_y, void* stream) {
    LQ_REQUIRE(N >= 0 && C >= 1 && H >= 1 && W >= 1 && Cout >= 1 && groups >= 1, "lq_conv2d_f32: bad shape");
    LQ_REQUIRE(C % groups == 0 && Cout % groups == 0, "lq_conv2d_f32: channels must divide by groups");
    LQ_REQUIRE(padding_mode >= LQ_PAD_ZEROS && padding_mode <= LQ_PAD_CIRCULAR, "lq_conv2d_f32: unknown padding mode");
    int64_t OH = 0, OW = 0;
    LQ_REQUIRE(conv_geometry(H, W, (int)KH, (int)KW, stride_h, stride_w, pad_top, pad_bottom, pad_left, pad_right,
                             dilation_h, dilation_w, &OH, &OW),
               "lq_conv2d_f32: kernel, stride, padding or dilation do not fit the input");
    if (padding_mode != LQ_PAD_ZEROS)
        LQ_REQUIRE(pad_top < H && pad_bottom < H && pad_left < W && pad_right < W,
                   "lq_conv2d_f32: reflect / replicate / circular padding must be smaller than the input");
    if (N == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_w && d_y, "lq_conv2d_f32: NULL pointer");
    LQ_REQUIRE(N * C * H * W < CV_MAX && N * Cout * OH * OW < CV_MAX, "lq_conv2d_f32: tensor too large");
    FConvArgs a{d_x, d_w, d_bias, d_y, (int)N, (int)C, (int)H, (int)W, (int)Cout, (int)groups, (int)(C / groups),
                (int)(Cout / groups), (int)KH, (int)KW, stride_h, stride_w, pad_top, pad_left, dilation_h, dilation_w,
                (int)OH, (int)OW, padding_mode};
    const int64_t total = N * Cout * OH * OW;
    hipLaunchKernelGGL(conv_f32_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, as_stream(stream), a);
    return launch_status("lq_conv2d_f32");
}

int lq_batch_norm_f32(const float* d_x, float* d_y, int64_t N, int64_t C, int64_t HW, const float* d_mean,
                      const float* d_var, const float* d_gamma, const float* d_beta, float eps, void* stream) {
    LQ_REQUIRE(N >= 0 && C >= 1 && HW >= 0 && N * C * HW < CV_MAX, "lq_batch_norm_f32: bad shape");
    if (N * HW == 0) return LQ_OK;
    LQ_REQUIRE(d_x && d_y && d_mean && d_var, "lq_batch_norm_f32: NULL pointer");
    const int64_t total = N * C * HW;
    hipLaunchKernelGGL(batch_norm_f32_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, as_stream(stream),
                       d_x, d_y, N, (int)C, HW, d_mean, d_var, d_gamma, d_beta, eps);
    return launch_status("lq_batch_norm_f32");
}

}  // extern "C"
