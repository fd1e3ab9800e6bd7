// lq_rnn.hip -- the element-wise step of the recurrent cells (RNN tanh / relu, LSTM, GRU).
//
// A recurrent layer's time step is two matrix products -- gx = x W_ih^T + b_ih (all time steps
// at once) and gh = h W_hh^T + b_hh (per step; the weight-only int8 GEMV for the dynamic
// modules) -- and this kernel, which combines them with the previous state in one pass:
//   RNN   h' = act(gx + gh)                                  (act = tanh or relu)
//   LSTM  g = gx + gh, gates (i, f, g, o) in that order;
//         c' = sigmoid(f) c + sigmoid(i) tanh(g);  h' = sigmoid(o) tanh(c')
//   GRU   r = sigmoid(gx_r + gh_r), z = sigmoid(gx_z + gh_z),
//         n = tanh(gx_n + r gh_n);  h' = (1 - z) n + z h
// (lucid/nn/modules/rnn.py: _rnn_step, _gru_step; the LSTM gate order of
// lucid/_C/nn/LSTM's lstm_forward).  sigmoid(x) = 1 / (1 + exp(-x)) as Lucid's sigmoid
// (backend/cpu/methods/Activation.cpp:8-50); exp / tanh are the device library's.  h' goes to
// h_next[B, H] and, when y is given, to row b of y with leading dimension ld_y (the layer's
// output sequence); c' (LSTM) to c_next.
#include <hip/hip_runtime.h>

#include "lq_internal.h"

namespace lq {

struct RnnArgs {
    int kind;
    const float* gx;
    int64_t ld_gx;
    const float* gh;
    int64_t ld_gh;
    const float* h;
    const float* c;
    int64_t B, H;
    float* h_next;
    float* c_next;
    float* y;
    int64_t ld_y;
};

__device__ __forceinline__ float rnn_sigmoid(float x) {
    const float e = expf(-x);
    const float d = 1.0f + e;
    return 1.0f / d;
}

__global__ __launch_bounds__(256) void rnn_cell_kernel(RnnArgs a) {
    const int64_t total = a.B * a.H;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t b = i / a.H, j = i - b * a.H;
        const float* gx = a.gx + b * a.ld_gx;
        const float* gh = a.gh + b * a.ld_gh;
        float hn;
        if (a.kind == LQ_RNN_TANH || a.kind == LQ_RNN_RELU) {
            const float pre = gx[j] + gh[j];
            hn = a.kind == LQ_RNN_TANH ? tanhf(pre) : ((pre <= 0.0f) ? 0.0f : pre);
        } else if (a.kind == LQ_RNN_LSTM) {
            const int64_t H = a.H;
            const float ig = rnn_sigmoid(gx[j] + gh[j]);
            const float fg = rnn_sigmoid(gx[H + j] + gh[H + j]);
            const float gg = tanhf(gx[2 * H + j] + gh[2 * H + j]);
            const float og = rnn_sigmoid(gx[3 * H + j] + gh[3 * H + j]);
            const float fc = fg * a.c[i];
            const float ic = ig * gg;
            const float cn = fc + ic;
            hn = og * tanhf(cn);
            a.c_next[i] = cn;
        } else {  // LQ_RNN_GRU
            const int64_t H = a.H;
            const float r = rnn_sigmoid(gx[j] + gh[j]);
            const float z = rnn_sigmoid(gx[H + j] + gh[H + j]);
            const float rn = r * gh[2 * H + j];
            const float n = tanhf(gx[2 * H + j] + rn);
            const float zc = 1.0f - z;
            const float a1 = zc * n;
            const float a2 = z * a.h[i];
            hn = a1 + a2;
        }
        a.h_next[i] = hn;
        if (a.y) a.y[b * a.ld_y + j] = hn;
    }
}

}  // namespace lq

using namespace lq;

extern "C" {

int lq_rnn_cell(int kind, const float* d_gx, int64_t ld_gx, const float* d_gh, int64_t ld_gh, const float* d_h,
                const float* d_c, int64_t B, int64_t H, float* d_h_next, float* d_c_next, float* d_y, int64_t ld_y,
                void* stream) {
    LQ_REQUIRE(kind >= LQ_RNN_TANH && kind <= LQ_RNN_GRU, "lq_rnn_cell: bad kind");
    LQ_REQUIRE(B >= 0 && H >= 0, "lq_rnn_cell: negative shape");
    if (B == 0 || H == 0) return LQ_OK;
    const int64_t G = kind == LQ_RNN_LSTM ? 4 : kind == LQ_RNN_GRU ? 3 : 1;
    LQ_REQUIRE(d_gx && d_gh && d_h_next, "lq_rnn_cell: NULL pointer");
    LQ_REQUIRE(ld_gx >= G * H && ld_gh >= G * H, "lq_rnn_cell: gate rows shorter than gates x H");
    LQ_REQUIRE(kind != LQ_RNN_LSTM || (d_c && d_c_next), "lq_rnn_cell: an LSTM step needs c and c_next");
    LQ_REQUIRE(kind != LQ_RNN_GRU || d_h, "lq_rnn_cell: a GRU step needs h");
    LQ_REQUIRE(!d_y || ld_y >= H, "lq_rnn_cell: ld_y < H");
    RnnArgs a{kind, d_gx, ld_gx, d_gh, ld_gh, d_h, d_c, B, H, d_h_next, d_c_next, d_y, ld_y};
    int64_t blocks = (B * H + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(rnn_cell_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), a);
    return launch_status("lq_rnn_cell");
}

}  // extern "C"
