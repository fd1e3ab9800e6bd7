/*
 * lq_api.h -- C ABI of the MI355X (gfx950) int8 quantized-inference backend.
 *
 * Every entry point is `extern "C"`, takes plain pointers and sizes, returns an
 * int status (LQ_OK == 0, negative on error; the message is in lq_last_error(),
 * thread-local) and never throws.  Compute entry points are asynchronous on the
 * HIP stream passed as `void* stream` (NULL = the null stream).  Device pointers
 * are marked `d_`; the caller owns every buffer.  Entry points that need
 * scratch memory take an explicit workspace whose size comes from the matching
 * `*_workspace_size` query.
 *
 * Reference seams this ABI replaces (paths relative to lucid-official/lucid):
 *   - the pybind op seam `_C_engine.quantized.{quantize,dequantize,quantized_matmul}`
 *     lucid/_C/bindings/bind_quantized.cpp:17-27, lucid/_C/engine.pyi:741-748,
 *     implemented by lucid/_C/ops/quantized/QuantizedMatmul.cpp:111-207;
 *   - the CPU backend calls the sidecar modules bottom out in
 *     (lucid/_C/backend/IBackend.h:228 via Dispatcher::for_device,
 *     lucid/_C/backend/Dispatcher.h:101-140): min/max reductions
 *     (backend/cpu/Reduce.cpp:54-135), round/clip/mul/add elementwise passes
 *     (methods/Unary.cpp:143-147, methods/Binary.cpp:24-104,481-523), the saturating
 *     float->int cast (methods/Factory.cpp:103-146), `linear` = sgemm + bias
 *     (methods/Matmul.cpp:80-122) and conv = im2col + sgemm (methods/Conv.cpp:271-360).
 *
 * Arithmetic contract (float32, no FMA contraction, round-half-to-even):
 *   quantize     c = satcast(clip(rne(fl32(x * inv)) + z, qmin, qmax))
 *   dequantize   y = fl32(fl32(float(c) - z) * s)
 *   fake-quant   y = fl32(fl32(clip(rne(fl32(x * inv)) + z, qmin, qmax) - z) * s)
 *   inv          = fl32(1.0f / s) when s comes from device memory (a tensor scale),
 *                  or the caller-supplied value (fl32(1.0 / double(s)) for a host scalar).
 *   following lucid/quantization/_functional.py:59-69,195-197,293,326-328.
 */
#ifndef LQ_API_H
#define LQ_API_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LQ_ABI_VERSION 1

/* ---- status codes -------------------------------------------------------- */
enum {
    LQ_OK = 0,
    LQ_ERR_INVALID = -1,     /* bad argument (shape, dtype, NULL pointer, alignment) */
    LQ_ERR_HIP = -2,         /* a HIP runtime call failed */
    LQ_ERR_UNSUPPORTED = -3, /* valid request this build does not implement */
    LQ_ERR_NOMEM = -4        /* device allocation failed */
};

/* ---- element types of code / output buffers ------------------------------ */
enum {
    LQ_I8 = 1,    /* int8 codes (qint8 / qint4 grids) */
    LQ_U8 = 2,    /* uint8 codes */
    LQ_I16 = 3,   /* int16 codes (Lucid stores quint8 as int16, _qscheme.py:243) */
    LQ_I32 = 4,   /* int32 (accumulators) */
    LQ_F16 = 5,   /* IEEE half */
    LQ_F32 = 6,   /* IEEE single */
    LQ_U8S8 = 7,  /* an unsigned-grid code c stored as int8 (c - 128): MFMA operand form */
    LQ_I64 = 8,   /* int64 (indices and offsets) */
    LQ_I8_QPAIR = 9, /* table lookups only: int8 rows whose d_scale holds interleaved float32
                      * {scale, zero point} pairs per row (d_zero_point unused) */
    LQ_BF16 = 10     /* bfloat16 (the upper 16 bits of a float32) */
};

/* ---- runtime -------------------------------------------------------------- */
/* Version of this ABI (LQ_ABI_VERSION).  No reference counterpart. */
int lq_abi_version(void);
/* Message of the last failed call on this thread ("" if none). */
const char* lq_last_error(void);
/* Kernel variant the last GEMM / convolution call on this thread launched, e.g.
 * "gemm dma 256x128" ("" before any).  Diagnostics for tests and profiles; no reference
 * counterpart. */
const char* lq_last_path(void);
/* Name of the backend ("hip-gfx950"); replaces the backend registration of
 * lucid/_C/backend/BackendInit.cpp:25-38. */
const char* lq_backend_name(void);
/* Number of visible HIP devices (0 when no GPU is present; not an error). */
int lq_device_count(int* count);
int lq_set_device(int device);
int lq_get_device(int* device);
/* Device allocations come from a per-device caching allocator (stands in for the engine
 * allocator, lucid/_C/core/Allocator.h, for device storage).  Stream contract:
 *   lq_free_async(p, s) returns p to the cache as last used on stream s (work already
 *   queued on s may still read or write it; no synchronisation).  lq_malloc_async(&p, n, s)
 *   hands out a cached block freed on s at once (s runs in order), and a block freed on
 *   another stream only after the work queued there before its free has completed (an
 *   event recorded at the free); otherwise it allocates.  A block freed on a stream under
 *   graph capture is reused on that stream only.  lq_malloc / lq_free are the same calls
 *   on the null stream.  lq_empty_cache releases every cached block back to HIP. */
int lq_malloc(void** d_ptr, size_t bytes);
int lq_free(void* d_ptr);
int lq_malloc_async(void** d_ptr, size_t bytes, void* stream);
int lq_free_async(void* d_ptr, void* stream);
/* Marks the live allocation d_ptr (as lq_malloc returned it) as used by work queued on
 * `stream` besides the stream it will be freed on: at its free a completion event is
 * recorded on `stream` too, and the block is handed out again -- on any stream -- only after
 * that work has completed.  For tensors read or written by a side stream (graph replays,
 * copies on their own stream).  No reference counterpart (Lucid's engine runs one stream);
 * the role of torch's Tensor.record_stream. */
int lq_record_stream(void* d_ptr, void* stream);
int lq_empty_cache(void);
/* Bytes currently handed out / held in the cache by the allocator. */
int lq_memory_stats(size_t* allocated, size_t* cached);
int lq_memcpy_h2d(void* d_dst, const void* h_src, size_t bytes, void* stream);
int lq_memcpy_d2h(void* h_dst, const void* d_src, size_t bytes, void* stream);
int lq_memcpy_d2d(void* d_dst, const void* d_src, size_t bytes, void* stream);
/* Fill `count` 32-bit words with `value` using a kernel (graph-capture safe). */
int lq_fill_u32(void* d_dst, uint32_t value, size_t count, void* stream);
/* The one-launch streaming-read floor the bandwidth-bound kernels are measured against: reads
 * `bytes` (a multiple of 16, 16-byte aligned) of d_src once, in 16 KB per workgroup, and
 * stores to d_sink[0..255] only when a thread's XOR of its words equals `never` (pick a value
 * that cannot occur, or give a 1 KB sink).  A measurement kernel with no counterpart in the
 * reference: Lucid's dispatch bench has no device floor to compare against. */
int lq_read_floor(const void* d_src, size_t bytes, uint32_t never, uint32_t* d_sink, void* stream);
int lq_stream_create(void** stream);
/* Waits for the stream's work, drops it from every allocation's lq_record_stream uses, then
 * destroys it. */
int lq_stream_destroy(void* stream);
int lq_stream_synchronize(void* stream);
int lq_device_synchronize(void);
int lq_event_create(void** event);
int lq_event_destroy(void* event);
int lq_event_record(void* event, void* stream);
int lq_event_synchronize(void* event);
int lq_event_elapsed_ms(float* ms, void* start, void* stop);
/* HIP graphs over a stream: capture the compute calls issued on `stream` between begin and
 * end into an executable graph, replay it without per-kernel host launch cost.  No
 * reference counterpart (Lucid's engine has no graph capture); for launch-bound callers
 * such as per-token decode.  Every compute entry point is capture-safe: none of them
 * allocates, memsets or synchronizes inside a call. */
int lq_graph_begin_capture(void* stream);
/* *graph_exec: an opaque handle owning the captured graph and its executable form, both
 * kept until lq_graph_destroy. */
int lq_graph_end_capture(void* stream, void** graph_exec);
int lq_graph_launch(void* graph_exec, void* stream);
int lq_graph_destroy(void* graph_exec);

/* ---- observers ------------------------------------------------------------ */
/* Observer update modes. */
enum {
    LQ_OBS_MINMAX = 0, /* running = minimum(running, batch) (MinMaxObserver, observer.py:408-414) */
    LQ_OBS_EMA = 1,    /* running = isinf(running_min) ? batch : running + c*(batch - running)
                          (MovingAverageMinMaxObserver, observer.py:527-544) */
    LQ_OBS_REPLACE = 2 /* running = batch (plain x.min()/x.max(), dynamic/linear.py:87) */
};

/* Per-tensor min/max of x[n] (NaN-propagating, -0 < +0, Reduce.cpp:54-105),
 * folded into the running 0-d buffers d_running_min / d_running_max by `mode`.  `ema_c` is the float32
 * averaging constant (LQ_OBS_EMA only).  n == 0 leaves the batch extrema at
 * {+inf, -inf}.  Two launches; workspace from lq_minmax_workspace_size. */
size_t lq_minmax_workspace_size(int64_t n);
int lq_minmax_f32(const float* d_x, int64_t n, float* d_running_min, float* d_running_max,
                  int mode, float ema_c, void* d_workspace, size_t workspace_bytes, void* stream);

/* Per-channel min/max of x viewed as [outer, C, inner] (channel axis in the
 * middle; PerChannelMinMaxObserver moveaxis+reshape+amin/amax, observer.py:672-685),
 * folded into d_running_min[C] / d_running_max[C] by `mode`.  For LQ_OBS_EMA the
 * seed test is "all of running_min is inf" (observer.py:1039-1044). */
size_t lq_minmax_per_channel_workspace_size(int64_t outer, int64_t C, int64_t inner);
int lq_minmax_per_channel_f32(const float* d_x, int64_t outer, int64_t C, int64_t inner,
                              float* d_running_min, float* d_running_max, int mode,
                              float ema_c, void* d_workspace, size_t workspace_bytes,
                              void* stream);

/* Histogram of x[n] over [lo, hi] in `bins` equal bins, Lucid's histc as HistogramObserver
 * calls it (lucid/quantization/observer.py:858-861 -> lucid/_ops/_adapters.py:1256-1279 ->
 * lucid/_C/backend/cpu/methods/Reduction.cpp:839-884): in double precision,
 * step = (hi - lo) / bins and v counts in bin trunc((v - lo) / step) (the top edge in the last
 * bin); values outside [lo, hi] and NaN are skipped.  d_hist[b] = float(count) (accumulate = 0)
 * or fl32(float(count) + d_hist[b]) (accumulate = 1: observer.py:863-865).  Needs hi > lo and
 * lq_histc_workspace_size(bins) bytes of workspace. */
size_t lq_histc_workspace_size(int64_t bins);
int lq_histc_f32(const float* d_x, int64_t n, int64_t bins, double lo, double hi, int accumulate,
                 float* d_hist, void* d_workspace, size_t workspace_bytes, void* stream);
/* HistogramObserver._rebin (lucid/quantization/observer.py:826-848): d_out[j] is the float32
 * sum, in source order, of d_hist[i] over the source bins i whose float32 center
 * old_min + (i + 0.5) * old_width lands, after (c - new_min) / new_width clipped to
 * [0, bins - 1] and truncated, on j.  old_width / new_width are the float32-rounded
 * (max - min) / bins.  bins <= 16384; d_out must not alias d_hist. */
int lq_hist_rebin_f32(const float* d_hist, int64_t bins, float old_min, float old_width,
                      float new_min, float new_width, float* d_out, void* stream);

/* calculate_qparams (lucid/quantization/_qparams.py:186-205) over n ranges:
 * scale[i], zero_point[i] from min[i], max[i].  symmetric != 0 selects the
 * symmetric branch; is_signed picks its zero point (0 or (qmax+qmin+1)//2). */
int lq_calc_qparams_f32(const float* d_min, const float* d_max, int64_t n, int symmetric,
                        int is_signed, int qmin, int qmax, float eps, float* d_scale,
                        float* d_zero_point, void* stream);

/* Dynamic per-tensor activation quantization: the live range of x[n] (MinMaxObserver in
 * replace mode), per-tensor affine qparams from it with eps (calculate_qparams,
 * lucid/quantization/_qparams.py:186-205) and the quantize of x onto them as codes q[n] of
 * q_dtype -- the activation step of the dynamic Linear, lucid/nn/quantized/dynamic/linear.py:
 * 85-92.  d_qparams[0..3] receive {min, max, scale, zero point}.  The same bits as
 * lq_minmax_f32 (LQ_OBS_REPLACE) -> lq_calc_qparams_f32 (asymmetric) ->
 * lq_quantize_per_tensor_f32 with the device scale; one launch for n <= 16384 (workspace
 * unused), those three otherwise (workspace of lq_dynamic_quantize_workspace_size(n) bytes). */
size_t lq_dynamic_quantize_workspace_size(int64_t n);
/* lq_layer_norm_f32 (d_res NULL) or lq_add_layer_norm_f32 (x += res written back first) on
 * rows x D, then lq_dynamic_quantize_f32 of the normalized rows into codes q [rows, D] and
 * d_qparams {min, max, scale, zero point}: one launch, the same bits (the normalized values
 * stay on chip).  The input step of a dynamic Linear after a LayerNorm (nn.LayerNorm ->
 * lucid/nn/quantized/dynamic/linear.py:85-92); rows * D <= 12288 (LQ_ERR_UNSUPPORTED above). */
int lq_layer_norm_quantize_f32(float* d_x, int64_t ldx, const float* d_res, int64_t ldres, int64_t rows, int64_t D,
                               const float* d_gamma, const float* d_beta, float ln_eps, int q_dtype, int qmin,
                               int qmax, float eps, float* d_qparams, void* d_q, void* stream);
int lq_dynamic_quantize_f32(const float* d_x, int64_t n, int q_dtype, int qmin, int qmax, float eps,
                            float* d_qparams, void* d_q, void* d_workspace, size_t workspace_bytes,
                            void* stream);
/* The same composition at any size, the normalized rows kept: lq_layer_norm_f32 (d_res NULL)
 * or lq_add_layer_norm_f32 (x += res written back first) into y [rows, D] (contiguous), then
 * lq_dynamic_quantize_f32 of y into codes q [rows, D] and d_qparams {min, max, scale, zero
 * point} -- the same bits as those calls.  Above 16384 values with a 16-byte aligned y and
 * codes aligned for four-code groups: two launches (the norm folds the extrema of what it
 * stores, the quantize folds the workgroups' pairs); otherwise the separate calls.  The input
 * step of a dynamic Linear after a LayerNorm (nn.LayerNorm -> lucid/nn/quantized/dynamic/
 * linear.py:85-92) at prefill sizes.  Workspace: lq_layer_norm_dynamic_quantize_workspace_size
 * bytes. */
size_t lq_layer_norm_dynamic_quantize_workspace_size(int64_t rows, int64_t D);
int lq_layer_norm_dynamic_quantize_f32(float* d_x, int64_t ldx, const float* d_res, int64_t ldres, int64_t rows,
                                       int64_t D, const float* d_gamma, const float* d_beta, float ln_eps, float* d_y,
                                       int q_dtype, int qmin, int qmax, float eps, float* d_qparams, void* d_q,
                                       void* d_workspace, size_t workspace_bytes, void* stream);

/* ---- quantize / dequantize / fake-quantize --------------------------------- */
/* Per-tensor quantize of x[n] to codes q[n] of type q_dtype (LQ_I8, LQ_U8,
 * LQ_I16, LQ_I32 or LQ_U8S8).  Scale: if d_scale != NULL the kernel uses
 * inv = fl32(1.0f / d_scale[0]); else inv = inv_scale_value.  Zero point:
 * d_zero_point[0] if non-NULL, else zero_point_value.
 * Replaces quantize(..., ch_axis=None), _functional.py:179-197. */
int lq_quantize_per_tensor_f32(const float* d_x, void* d_q, int64_t n, int q_dtype,
                               const float* d_scale, const float* d_zero_point,
                               float inv_scale_value, float zero_point_value, int qmin,
                               int qmax, void* stream);
/* Per-channel quantize, x viewed as [outer, C, inner]; inv = fl32(1.0f/scale[c]),
 * zero point d_zero_point[c] (or zero_point_value if NULL).
 * Replaces quantize(..., ch_axis=k) with _reshape_for_channel, _functional.py:47-56,190-197. */
int lq_quantize_per_channel_f32(const float* d_x, void* d_q, int64_t outer, int64_t C,
                                int64_t inner, int q_dtype, const float* d_scale,
                                const float* d_zero_point, float zero_point_value, int qmin,
                                int qmax, void* stream);
/* Per-tensor dequantize of codes q[n] (q_dtype LQ_I8/LQ_U8/LQ_I16/LQ_I32/LQ_U8S8)
 * to y[n] of y_dtype LQ_F32 or LQ_F16 (fl16 of the float32 result).
 * s = d_scale[0] or scale_value; z = d_zero_point[0] or zero_point_value.
 * Replaces dequantize(..., ch_axis=None), _functional.py:281-293. */
int lq_dequantize_per_tensor(const void* d_q, int q_dtype, void* d_y, int y_dtype, int64_t n,
                             const float* d_scale, const float* d_zero_point, float scale_value,
                             float zero_point_value, void* stream);
/* Per-channel dequantize ([outer, C, inner]); replaces dequantize(..., ch_axis=k). */
int lq_dequantize_per_channel(const void* d_q, int q_dtype, void* d_y, int y_dtype,
                              int64_t outer, int64_t C, int64_t inner, const float* d_scale,
                              const float* d_zero_point, float zero_point_value, void* stream);
/* Per-tensor fake-quantize forward (_FakeQuantizeAffine.forward, _functional.py:314-333):
 * y = fl32(fl32(clip(rne(fl32(x*inv)) + z) - z) * s).  With d_scale == NULL the
 * caller passes both inv_scale_value and scale_value.  d_mask (may be NULL)
 * receives the straight-through mask as float 1/0 (_functional.py:330-332). */
int lq_fake_quantize_per_tensor_f32(const float* d_x, float* d_y, int64_t n,
                                    const float* d_scale, const float* d_zero_point,
                                    float inv_scale_value, float scale_value,
                                    float zero_point_value, int qmin, int qmax, float* d_mask,
                                    void* stream);
/* Per-channel fake-quantize ([outer, C, inner]). */
int lq_fake_quantize_per_channel_f32(const float* d_x, float* d_y, int64_t outer, int64_t C,
                                     int64_t inner, const float* d_scale,
                                     const float* d_zero_point, float zero_point_value, int qmin,
                                     int qmax, float* d_mask, void* stream);

/* ---- W8A8 int8 GEMM with fused requantize epilogue -------------------------- */
/* Epilogue output kinds of lq_gemm_w8a8. */
enum {
    LQ_OUT_I32 = 0,  /* raw int32 accumulator */
    LQ_OUT_F32 = 1,  /* y */
    LQ_OUT_F16 = 2,  /* fl16(y) */
    LQ_OUT_Q8 = 3,   /* codes of y on the output grid, stored int8 (signed grid) */
    LQ_OUT_QU8 = 4,  /* codes of y on the output grid, stored uint8 (unsigned grid) */
    LQ_OUT_FQ32 = 5, /* fake-quantized y on the output grid, float32 (the sidecar module output) */
    LQ_OUT_Q16 = 6,  /* codes of y on the output grid, stored int16 (Lucid quint8 storage) */
    LQ_OUT_QU8S8 = 7 /* unsigned-grid codes c of y stored as int8 (c - 128): the next layer's
                        MFMA operand (LQ_U8S8) */
};
/* Flag bits of lq_gemm_w8a8.  LQ_EPI_A_U8S8: A holds unsigned-grid codes c stored as int8
 * (c - 128, the LQ_U8S8 form); d_a_zero_point (NULL = 0) is the grid's own zero point and
 * the kernel applies the 128 shift. */
enum { LQ_EPI_RELU = 1, LQ_EPI_A_U8S8 = 2, LQ_EPI_ROUND_BF16 = 4 /* lq_group_matmul only */,
       LQ_EPI_GELU = 8 /* lq_gemm_w8a8(_packed), LQ_OUT_F32 only: y = gelu_tanh(y) after the bias,
                          the bits of lq_gelu_tanh_f32 on the output (F.gelu after the Linear) */,
       LQ_CONV_OUT_NHWC = 16 /* lq_conv2d_i8 only, byte codes out, groups 1, Cout a multiple of 16:
                                y written [N][OH][OW][Cout] (the layout of lq_conv2d_i8_nhwc without a
                                border), the same codes */ };

/* C[m,n] epilogue of acc[m,n] = sum_k (A[m,k] - za) * (B[n,k] - zb[n])  (exact int32),
 * A int8 [M,K] row-major (lda), B int8 [N,K] row-major (ldb; Lucid's weight_int8 [out,in]).
 *   s  = fl32(a_scale[m * a_scale_stride] * b_scale[n * b_scale_stride])   (NULL scale = 1)
 *   y  = fl32(float(acc) * s); y = fl32(y + bias[n]) (bias may be NULL); ReLU if flagged
 *        (y <= 0 -> +0, NaN passes; Vdsp.cpp vrelu_f32);
 *   out by out_kind, requantized with inv = fl32(1.0f / out_scale[0]), z = out_zp[0]
 *   (c = clip(rne(fl32(y * inv)) + z, out_qmin, out_qmax), saturating store).
 * za = d_a_zero_point[0] (integer-valued float, NULL = 0); zb = d_b_zero_point[n] (NULL = 0).
 * The zero points enter as sum_k A*B - za*bsum[n] - zb[n]*asum[m] + K*za*zb[n] with
 * bsum[n] = sum_k B[n,k] (d_b_sums, e.g. cached by the module from lq_row_sums_i8; NULL =
 * computed into the workspace) and asum[m] = sum_k A[m,k] (computed when zb is given).
 * Fast paths need 16-byte aligned A/B, lda/ldb/K multiples of 16; other shapes run a
 * generic kernel with the same results.
 * Replaces the nnq.Linear / nnqd.Linear compute: dequantize(W) -> F.linear -> act ->
 * fake_quantize (lucid/nn/quantized/linear.py:206-215, dynamic/linear.py:85-92,
 * Linear.cpp:199 -> Matmul.cpp:80-122).  The workspace (lq_gemm_w8a8_workspace_size)
 * holds the code sums and, for mid-size M, split-K partial sums; with a smaller (or NULL)
 * workspace the call still succeeds when no zero-point sums must be computed, without split-K. */
size_t lq_gemm_w8a8_workspace_size(int64_t M, int64_t N, int64_t K);
int lq_gemm_w8a8(const int8_t* d_A, int64_t lda, const int8_t* d_B, int64_t ldb, void* d_C,
                 int64_t ldc, int64_t M, int64_t N, int64_t K, const float* d_a_scale,
                 int64_t a_scale_stride, const float* d_b_scale, int64_t b_scale_stride,
                 const float* d_a_zero_point, const float* d_b_zero_point,
                 const int32_t* d_b_sums, const float* d_bias, const float* d_out_scale,
                 const float* d_out_zero_point, int out_qmin, int out_qmax, int out_kind,
                 int flags, void* d_workspace, size_t workspace_bytes, void* stream);
/* lq_gemm_w8a8 without a workspace argument, allocating nothing: the code sums, split-K
 * partials and tile counters live in a static 16 MiB device array the library holds on each
 * GPU it runs on (lq_gemm_w8a8_noalloc_scratch_bytes()).  Shapes whose workspace
 * (lq_gemm_w8a8_workspace_size) exceeds it fail with LQ_ERR_UNSUPPORTED.  Calls on one GPU
 * share the array, so calls that overlap on one GPU (concurrent streams or threads) race;
 * serialize them.  Same results as lq_gemm_w8a8.  No counterpart in the reference: for
 * callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). */
size_t lq_gemm_w8a8_noalloc_scratch_bytes(void);
int lq_gemm_w8a8_noalloc(const int8_t* d_A, int64_t lda, const int8_t* d_B, int64_t ldb, void* d_C,
                         int64_t ldc, int64_t M, int64_t N, int64_t K, const float* d_a_scale,
                         int64_t a_scale_stride, const float* d_b_scale, int64_t b_scale_stride,
                         const float* d_a_zero_point, const float* d_b_zero_point,
                         const int32_t* d_b_sums, const float* d_bias, const float* d_out_scale,
                         const float* d_out_zero_point, int out_qmin, int out_qmax, int out_kind,
                         int flags, void* stream);
/* lq_gemm_w8a8 with float32 output y [M, N] (contiguous; bias, LQ_EPI_GELU / LQ_EPI_RELU /
 * LQ_EPI_A_U8S8 as there), then lq_dynamic_quantize_f32 of y into codes [M N] and d_qparams
 * {min, max, scale, zero point}: a dynamic Linear's product followed by the next dynamic
 * Linear's input step (lucid/nn/quantized/dynamic/linear.py:85-92), the same bits as the two
 * calls.  Where the product takes an LDS-DMA kernel with at most 1024 workgroups (and y and the
 * codes are aligned), its epilogue folds the extrema of what it stores per workgroup and the
 * quantize folds those pairs: two launches where the calls take three.  Workspace:
 * lq_gemm_w8a8_dynamic_quantize_workspace_size bytes (the product's workspace first). */
size_t lq_gemm_w8a8_dynamic_quantize_workspace_size(int64_t M, int64_t N, int64_t K);
int lq_gemm_w8a8_dynamic_quantize(const int8_t* d_A, int64_t lda, const int8_t* d_B, int64_t ldb, float* d_y,
                                  int64_t M, int64_t N, int64_t K, const float* d_a_scale, int64_t a_scale_stride,
                                  const float* d_b_scale, int64_t b_scale_stride, const float* d_a_zero_point,
                                  const float* d_b_zero_point, const int32_t* d_b_sums, const float* d_bias, int flags,
                                  int q_dtype, int qmin, int qmax, float eps, float* d_qparams, void* d_codes,
                                  void* d_workspace, size_t workspace_bytes, void* stream);
/* ---- MFMA-packed weights for decode (M <= 128) ------------------------------ */
/* Bytes of the packed form of an int8 weight B [N, K]: ceil(N/16) x ceil(K/64) tiles of
 * 1 KB.  Tile (t, s) sits at byte (t * ceil(K/64) + s) * 1024; its 16-byte chunk l holds
 * row 16 t + l % 16, K-bytes 64 s + 16 (l / 16) .. +15 (zero past N and K), i.e. the
 * A-operand fragment of v_mfma_i32_16x16x64_i8, so a wave load is 1 KB contiguous.
 * No reference counterpart: a device layout of Lucid's weight_int8 [out, in]
 * (lucid/nn/quantized/linear.py:183-199), which stays the state_dict form. */
size_t lq_packed_weights_size(int64_t N, int64_t K);
int lq_pack_weights_i8(const int8_t* d_B, int64_t ldb, int64_t N, int64_t K, int8_t* d_packed,
                       void* stream);
/* lq_gemm_w8a8 with B in the packed form, for M <= 128 (decode); LQ_ERR_UNSUPPORTED above.
 * Needs K and lda multiples of 16, 16-byte aligned A and packed B, and the cached weight
 * sums d_b_sums whenever d_a_zero_point is given.  Same results as lq_gemm_w8a8. */
int lq_gemm_w8a8_packed(const int8_t* d_A, int64_t lda, const int8_t* d_B_packed, void* d_C,
                        int64_t ldc, int64_t M, int64_t N, int64_t K, const float* d_a_scale,
                        int64_t a_scale_stride, const float* d_b_scale, int64_t b_scale_stride,
                        const float* d_a_zero_point, const float* d_b_zero_point,
                        const int32_t* d_b_sums, const float* d_bias, const float* d_out_scale,
                        const float* d_out_zero_point, int out_qmin, int out_qmax, int out_kind,
                        int flags, void* d_workspace, size_t workspace_bytes, void* stream);

/* nnqd.Linear's whole forward at decode sizes in one launch, with the float module before it
 * folded in: the input a [M, K] is
 *   src LQ_DL_PLAIN   a = x
 *       LQ_DL_LN      a = layer_norm(x)                      (the bits of lq_layer_norm_f32)
 *       LQ_DL_ADD_LN  s = x + res, a = layer_norm(s)         (lq_add_layer_norm_f32; s is
 *                     stored to d_sum when it is not NULL -- a buffer other than x, which
 *                     stays as it was)
 * (gamma / beta NULL: 1 / 0), then the live min / max of all M x K values, the per-tensor affine
 * qparams on the unsigned grid [qmin, qmax] (0 <= qmin < qmax <= 255; stored to d_qparams as
 * {min, max, scale, zero point} when not NULL), the codes of lq_dynamic_quantize_f32, and the
 * float32 product of lq_gemm_w8a8_packed (LQ_EPI_A_U8S8) with the packed weight, its per-row
 * scales and code sums and the bias; flags 0 or LQ_EPI_GELU.  The bits of those launches in
 * sequence.  For M <= 16, K a multiple of 16, M K <= 16384 (with a norm: K <= 2048 and
 * M K <= 8192), x rows 16-byte aligned without a norm; LQ_ERR_UNSUPPORTED otherwise.
 * Replaces, as one call, the steps of Lucid's dynamic Linear forward
 * (lucid/nn/quantized/dynamic/linear.py:85-92: calculate_qparams of x.min() / x.max(),
 * fake_quantize, the linear) and the LayerNorm module that precedes it in a decoder. */
enum { LQ_DL_PLAIN = 0, LQ_DL_LN = 1, LQ_DL_ADD_LN = 2 };
int lq_dynamic_linear_packed_f32(const float* d_x, int64_t ldx, const float* d_res, int64_t ldres, float* d_sum,
                                 int64_t ld_sum, int src, const float* d_gamma, const float* d_beta, float ln_eps,
                                 int64_t M, int64_t K, int qmin, int qmax, float eps, float* d_qparams,
                                 const int8_t* d_w_packed, const float* d_w_scale, const int32_t* d_w_sums,
                                 const float* d_bias, int64_t N, float* d_y, int64_t ldy, int flags, void* stream);

/* sums[r] = sum_k X[r,k] over int8 rows (the weight code sums a module caches for the
 * activation zero-point correction).  No reference counterpart (Lucid has no integer GEMM). */
int lq_row_sums_i8(const int8_t* d_X, int64_t ld, int64_t rows, int64_t K, int32_t* d_sums,
                   void* stream);

/* ---- weight-only int8 GEMV / skinny GEMM -------------------------------------------- */
/* y[m,n] = w_scale[n] * (sum_k W[n,k] x[m,k] - zb[n] sum_k x[m,k]) + bias[n] (ReLU with
 * LQ_EPI_RELU): Lucid's sidecar Linear on a float input, dequantize -> F.linear
 * (lucid/nn/quantized/linear.py:206-210 -> lucid/_C/nn/Linear.cpp:199), without forming
 * the float weight.  x / y of x_dtype (LQ_F32 or LQ_F16), W int8 [N, ldw] row-major,
 * d_w_zero_point / d_bias may be NULL.  Float32 accumulation (tolerance parity: the float
 * GEMM's summation order is the reference's own).  Any M; tuned for M <= 16.  With
 * lq_gemv_w8_workspace_size(M, N, K) bytes of device workspace (16-byte aligned; 0 for M <= 2)
 * float32 activations of M > 8 rows are split into fp16 halves once per call instead of once
 * per workgroup (for fewer rows the in-workgroup split is faster and the workspace is not
 * touched); without it (NULL) the call still runs, with identical results. */
size_t lq_gemv_w8_workspace_size(int64_t M, int64_t N, int64_t K);
int lq_gemv_w8(const void* d_x, int x_dtype, int64_t ldx, const int8_t* d_W, int64_t ldw,
               const float* d_w_scale, const float* d_w_zero_point, const float* d_bias,
               void* d_y, int64_t ldy, int64_t M, int64_t N, int64_t K, int flags,
               void* d_workspace, size_t workspace_bytes, void* stream);
/* lq_gemv_w8 for decode (1 <= M <= 16) over the MFMA-packed weight of lq_pack_weights_i8 (the
 * copy lq_gemm_w8a8_packed reads), so each wave loads 1 KB of consecutive weight bytes.  Same
 * arithmetic and arguments as lq_gemv_w8 without ldw; K a positive multiple of 16; x, its rows
 * and the packed weight 16-byte aligned; lq_gemv_w8_packed_workspace_size(M, N, K) bytes of
 * workspace (0 when K <= 512).  Replaces the same seam as lq_gemv_w8
 * (lucid/nn/quantized/linear.py:206-210) for the layer's decode calls. */
size_t lq_gemv_w8_packed_workspace_size(int64_t M, int64_t N, int64_t K);
int lq_gemv_w8_packed(const void* d_x, int x_dtype, int64_t ldx, const int8_t* d_W_packed,
                      const float* d_w_scale, const float* d_w_zero_point, const float* d_bias, void* d_y,
                      int64_t ldy, int64_t M, int64_t N, int64_t K, int flags, void* d_workspace,
                      size_t workspace_bytes, void* stream);

/* ---- group-wise packed weights (QuantizedLinearMLX layout) -------------------------- */
/* Group-wise affine quantize of W[N,K] (float32) with groups of group_size (32/64/128) along K:
 * s_g = (max_g - min_g) / (2^bits - 1), b_g = min_g, c = clip(rne((w - b_g) / s_g), 0, 2^bits-1)
 * (codes 0 when s_g is not > 0), 32/bits codes per uint32 little-end first.  packed
 * [N, K*bits/32] uint32, scales/biases [N, K/group_size] float32.  Replaces
 * _C_engine.quantized.quantize (lucid/_C/bindings/bind_quantized.cpp:17-27 ->
 * lucid/_C/ops/quantized/QuantizedMatmul.cpp:111-121; formula lucid/quantization/_qgemm.py:84-97). */
int lq_group_quantize_f32(const float* d_w, int64_t N, int64_t K, int group_size, int bits,
                          uint32_t* d_packed, float* d_scales, float* d_biases, void* stream);
/* w_hat = fl32(fl32(c * s_g) + b_g) as float32 [N, K] (d_biases NULL: b_g = 0).  Replaces
 * _C_engine.quantized.dequantize (QuantizedMatmul.cpp:123-141, _qgemm.py:167-170). */
int lq_group_dequantize_f32(const uint32_t* d_packed, const float* d_scales,
                            const float* d_biases, int64_t N, int64_t K, int group_size,
                            int bits, float* d_w, void* stream);
/* y[m,n] = sum_k x[m,k] w_hat[n,k] (+ bias[n]) (ReLU with LQ_EPI_RELU), x / y of x_dtype
 * (LQ_F32 or LQ_F16), float32 accumulation, without forming w_hat.  Replaces
 * _C_engine.quantized.quantized_matmul (QuantizedMatmul.cpp:143-163) for transpose = 1.
 * Dtype rule of the reference: scales and group biases are cast to x's dtype before the
 * product (QuantizedMatmul.cpp:153-164) and the result is x's dtype; QuantizedLinearMLX then
 * adds its bias cast to that dtype (mlx_linear.py:215-222).  So with LQ_F16 x the scales,
 * group biases and bias are rounded to half, the float32 sum is rounded to half, and the
 * bias is added in half.  LQ_EPI_ROUND_BF16 (float32 x and y only) applies the same rule
 * for bfloat16: a caller with bfloat16 activations widens x to float32 (exact, lq_cast),
 * calls with this flag and narrows y (exact: y is bfloat16-valued).
 * transpose = 0: y[m,k] = sum_n x[m,n] w_hat[n,k] (+ bias[k]) with x [M, N] (ldx >= N) and
 * y [M, K] (ldy >= K), w_hat tiles dequantized as lq_group_dequantize_f32 writes them -- the
 * transpose=false product and the QLoRA input gradient dX = dY dequant(W) of the transpose=1
 * product (QuantizedMatmulBackward::apply, QuantizedMatmul.cpp:73-90); no workspace.
 * d_biases (group offsets) and d_bias (layer bias) may be NULL.
 * lq_group_matmul_workspace_size(M, N, K, group_size) bytes of workspace let float32
 * activations be split once per call for transpose = 1 (as for lq_gemv_w8; NULL still runs). */
size_t lq_group_matmul_workspace_size(int64_t M, int64_t N, int64_t K, int group_size);
int lq_group_matmul(const void* d_x, int x_dtype, int64_t ldx, const uint32_t* d_packed,
                    const float* d_scales, const float* d_biases, const float* d_bias, void* d_y,
                    int64_t ldy, int64_t M, int64_t N, int64_t K, int group_size, int bits,
                    int transpose, int flags, void* d_workspace, size_t workspace_bytes,
                    void* stream);

/* ---- quantizable merges (FloatFunctional / QFunctional) ------------------------- */
/* Operations of lq_qmerge. */
enum { LQ_MERGE_ADD = 0, LQ_MERGE_MUL = 1, LQ_MERGE_ADD_SCALAR = 2, LQ_MERGE_MUL_SCALAR = 3, LQ_MERGE_COPY = 4 };
/* Element-wise merge over a rows x cols block, the ops of FloatFunctional and QFunctional
 * (lucid/nn/quantized/functional_module.py:95-120 and 195-229: add, mul, add_scalar,
 * mul_scalar, add_relu = add with LQ_EPI_RELU, cat = LQ_MERGE_COPY into a slice).
 * Operand a (and b for ADD / MUL) is read contiguously as float32 (type LQ_F32) or as codes
 * (LQ_I8 / LQ_U8 / LQ_I16 / LQ_U8S8) with a per-tensor grid: value fl32(fl32(float(c) - z) * s)
 * (d_*_scale required, d_*_zero_point NULL = 0).  t = a + b, a * b, a + scalar, a * scalar or
 * a, one float32 operation, then ReLU (y <= 0 -> +0) with LQ_EPI_RELU.  out_type LQ_F32 stores
 * t; a code type stores the codes of t on [qmin, qmax] with d_out_scale / d_out_zero_point
 * (QFunctional's fake-quantize grid: clip(rne(t * fl32(1 / S)) + Z), NaN -> 0).  Element
 * (r, c) goes to d_out[r * ld_out + c].  No reference counterpart for the fused form: Lucid
 * runs the float op, then fake_quantize (functional_module.py:188-229). */
int lq_qmerge(int op, const void* d_a, int a_type, const float* d_a_scale, const float* d_a_zero_point,
              const void* d_b, int b_type, const float* d_b_scale, const float* d_b_zero_point, float scalar,
              int64_t rows, int64_t cols, int64_t ld_out, const float* d_out_scale,
              const float* d_out_zero_point, int qmin, int qmax, int flags, int out_type, void* d_out,
              void* stream);

/* ---- activations (float and quantized) ------------------------------------------ */
/* Activations of lq_qact. */
enum { LQ_ACT_SIGMOID = 0, LQ_ACT_TANH = 1, LQ_ACT_HARDSWISH = 2, LQ_ACT_HARDSIGMOID = 3, LQ_ACT_ELU = 4,
       LQ_ACT_LEAKY_RELU = 5 };
/* y[i] = act(x[i]) over n contiguous elements: the float activations F.sigmoid / tanh /
 * hardswish / hardsigmoid / elu / leaky_relu (lucid/_C/backend/cpu/methods/Activation.cpp:8-50,
 * 375-460, 661-751; Unary.cpp:165-170) with out_type LQ_F32, and the quantized activations
 * nnq.Sigmoid / Tanh / Hardswish / Hardsigmoid / ELU / LeakyReLU
 * (lucid/nn/quantized/activation.py:20-475: the activation, then fake-quantize) with a code
 * out_type (LQ_I8 / LQ_U8 / LQ_I16 / LQ_U8S8) on [qmin, qmax] with d_out_scale /
 * d_out_zero_point (clip(rne(t * fl32(1 / S)) + Z), NaN -> 0).  param is ELU's alpha or
 * LeakyReLU's negative_slope (as float32), ignored otherwise.  x is float32 (LQ_F32) or codes
 * with a per-tensor grid, read as fl32(fl32(float(c) - z) * s) (d_x_scale required,
 * d_x_zero_point NULL = 0).  Replaces _C_engine.sigmoid / tanh / hard_swish / hard_sigmoid /
 * elu / leaky_relu (lucid/nn/functional/activations.py:99-579) followed, for the quantized
 * modules, by the fake-quantize of _QuantizedGridModule (lucid/nn/quantized/_utils.py:29-45). */
int lq_qact(int op, const void* d_x, int x_type, const float* d_x_scale, const float* d_x_zero_point,
            int64_t n, float param, const float* d_out_scale, const float* d_out_zero_point, int qmin,
            int qmax, int out_type, void* d_y, void* stream);

/* ---- table lookups (Embedding / EmbeddingBag) ----------------------------------- */
/* Pooling modes of lq_embedding_bag (the engine's encoding, lucid/nn/functional/sparse.py:214). */
enum { LQ_BAG_SUM = 0, LQ_BAG_MEAN = 1, LQ_BAG_MAX = 2 };
/* out[i, :] = row idx[i] of a [rows, D] table: int8 codes (table_type LQ_I8) dequantized per row
 * as fl32(fl32(float(c) - z[r]) * s[r]) (d_zero_point NULL = 0), the same with the row's
 * {s, z} read as one pair from d_scale (LQ_I8_QPAIR: one random cache line per lookup fewer),
 * or float32 entries (LQ_F32, d_scale unused).  Indices LQ_I32 or LQ_I64; one outside [0, rows) gives a NaN row (no read).
 * Replaces dequantize(table, ch_axis=0) + F.embedding of nnq.Embedding.forward
 * (lucid/nn/quantized/sparse.py:140-143 -> lucid/_C/backend/cpu/methods/Sequence.cpp:520-552),
 * and the float lookup of nn.Embedding, without forming the float table. */
int lq_embedding(const void* d_table, int table_type, const float* d_scale, const float* d_zero_point,
                 int64_t rows, int64_t D, const void* d_idx, int idx_type, int64_t n_idx, float* d_out,
                 void* stream);
/* Pooled lookup into out[n_bags, D] (float32).  Bags: with d_offsets (LQ_I32 / LQ_I64,
 * n_offsets entries) bag b = [off[b], off[b + 1]) and the last runs to n_idx, or to
 * off[n_offsets - 1] with include_last_offset (then n_bags = n_offsets - 1); without, fixed
 * bags of bag_len (a 2-D input, one bag per row).  Each bag walks its indices in order:
 * LQ_BAG_SUM acc = acc + v, LQ_BAG_MEAN the sum / count, LQ_BAG_MAX acc = v > acc ? v : acc
 * from the lowest float (an empty bag is 0).  Indices equal to padding_idx (-1 = none) are
 * skipped and not counted.  d_per_sample_weights (LQ_BAG_SUM only) adds fl32(v * w[k]) instead,
 * a padding index adding fl32(v * 0).  An index outside [0, rows) makes its bag NaN.  Offsets
 * are clamped to [0, n_idx] (the caller validates them).  Replaces nnq.EmbeddingBag.forward
 * (lucid/nn/quantized/sparse.py:284-304 -> lucid/_C/backend/cpu/methods/Sequence.cpp:8-93, and
 * the per_sample_weights composite lucid/nn/functional/sparse.py:228-310). */
int lq_embedding_bag(const void* d_table, int table_type, const float* d_scale, const float* d_zero_point,
                     int64_t rows, int64_t D, const void* d_idx, int idx_type, int64_t n_idx,
                     const void* d_offsets, int offsets_type, int64_t n_offsets, int include_last_offset,
                     int64_t bag_len, int mode, int64_t padding_idx, const float* d_per_sample_weights,
                     float* d_out, void* stream);

/* ---- recurrent cells --------------------------------------------------------------- */
enum { LQ_RNN_TANH = 0, LQ_RNN_RELU = 1, LQ_RNN_LSTM = 2, LQ_RNN_GRU = 3 };
/* One time step of B rows of a recurrent cell from its two gate products gx[b, :] = x W_ih^T +
 * b_ih (row stride ld_gx) and gh[b, :] = h W_hh^T + b_hh (row stride ld_gh), G x H wide (G = 1,
 * 4 for LSTM gates i, f, g, o, 3 for GRU gates r, z, n):
 *   RNN  h' = tanh / relu(gx + gh);  LSTM  c' = s(f) c + s(i) tanh(g), h' = s(o) tanh(c');
 *   GRU  r = s(gx_r + gh_r), z = s(gx_z + gh_z), n = tanh(gx_n + r gh_n), h' = (1 - z) n + z h
 * with s(x) = 1 / (1 + exp(-x)) (lucid/nn/modules/rnn.py _rnn_step / _gru_step, the LSTM of
 * lstm_forward).  h / c / h_next / c_next are [B, H] contiguous (h_next may be h, c_next may be
 * c); h' is also written to d_y[b * ld_y + j] when d_y is not NULL.  The step the float and
 * the dynamic int8 LSTM / GRU / cells (lucid/nn/quantized/dynamic/rnn.py) share. */
int lq_rnn_cell(int kind, const float* d_gx, int64_t ld_gx, const float* d_gh, int64_t ld_gh, const float* d_h,
                const float* d_c, int64_t B, int64_t H, float* d_h_next, float* d_c_next, float* d_y, int64_t ld_y,
                void* stream);

/* ---- transposed convolution ------------------------------------------------------- */
/* y[p, h, w] = x[p, h / stride_h, w / stride_w] where both divide, else the zero value, over
 * `planes` planes of H x W -> ((H - 1) stride_h + 1) x ((W - 1) stride_w + 1): the expanded
 * input that turns conv_transpose2d into a stride-1 convolution (padding d (k - 1) - p, the
 * kernel flipped with its channel axes swapped).  elem_type LQ_F32 (zero value 0.0) or
 * LQ_I8 / LQ_U8S8 codes (zero value: the code of d_zero_point[0], NULL = 0).  Replaces the
 * stride handling of F.conv_transpose2d under nnq.ConvTranspose2d
 * (lucid/nn/quantized/conv_transpose.py:146-175); no reference counterpart as an op. */
int lq_stride_expand(const void* d_x, int elem_type, int64_t planes, int64_t H, int64_t W, int stride_h,
                     int stride_w, const float* d_zero_point, void* d_y, void* stream);
/* The depth gather of a 3-D convolution run as a 2-D one: x [N, C, D, HW] (elements LQ_F32,
 * or int8 codes LQ_I8 / LQ_U8S8) -> y [N OD, groups, KD, C / groups, HW], where output depth od
 * reads input depth e = od stride - pad + kd dilation for kernel depth kd; out-of-range
 * depths (pad_mode 0), and with expand > 1 the depths e % expand != 0 of a transposed
 * convolution's stride-expanded axis (e / expand otherwise), hold the zero value (the zero
 * point code read from d_zero_point for codes, minus 128 for LQ_U8S8; 0.0 for floats);
 * pad_mode 1 / 2 / 3 map them reflect / replicate / circular (expand 1).  The 3-D layers of
 * lucid/nn/quantized/conv.py:491 (Conv3d), intrinsic.py:344 (ConvReLU3d) and
 * conv_transpose.py:473 (ConvTranspose3d) and their float modules run on the 2-D
 * implicit-GEMM convolution this way; no reference counterpart as an op. */
int lq_depth_gather(const void* d_x, int elem_type, int64_t N, int64_t C, int64_t D, int64_t HW, int64_t groups,
                    int64_t KD, int64_t OD, int64_t stride, int64_t pad, int64_t dilation, int64_t expand,
                    int pad_mode, const float* d_zero_point, void* d_y, void* stream);
/* y[a][c][b][p] = x[a][b][c][p] for elements of 1, 2 or 4 bytes (y must not alias x): the
 * 2-D convolution's [N, OD, Cout, OH OW] output back to NCDHW, and kernels into the gathered
 * channel order. */
int lq_permute_0213(const void* d_x, int elem_bytes, int64_t A, int64_t B, int64_t C, int64_t P, void* d_y,
                    void* stream);

/* ---- pooling ---------------------------------------------------------------------- */
enum { LQ_POOL_MAX = 0, LQ_POOL_AVG = 1 };
enum { LQ_POOL_ADAPTIVE = 1, LQ_POOL_COUNT_INCLUDE_PAD = 2 };
/* 2-D pooling of x[N, C, H, W] into y[N, C, OH, OW] (NCHW, contiguous).  Windows: KH x KW at
 * stride (stride_h, stride_w) with implicit padding (pad at most half the window; OH / OW as
 * floor((H + 2 pad - K) / stride) + 1), or with LQ_POOL_ADAPTIVE the cells
 * [floor(o S / O), ceil((o + 1) S / O)) of an adaptive pool.  LQ_POOL_MAX: the first
 * in-window element replaced by any greater one or by a NaN (padding skipped); y has x's
 * element type, and a code input stays on its grid (codes compare as their values).
 * LQ_POOL_AVG: float32 sum in row-major window order divided by the window size (with
 * LQ_POOL_COUNT_INCLUDE_PAD the padded size), y float32; a code input (LQ_I8 / LQ_U8 / LQ_I16 /
 * LQ_U8S8) is read as fl32(fl32(float(c) - z) * s).  Replaces max_pool2d / avg_pool2d /
 * adaptive_avg_pool2d (lucid/_C/backend/cpu/Pool.cpp:27-168,
 * lucid/nn/functional/_pool_core.py:228-250, 407-434). */
int lq_pool2d(int op, const void* d_x, int x_type, const float* d_x_scale, const float* d_x_zero_point, int64_t N,
              int64_t C, int64_t H, int64_t W, int64_t OH, int64_t OW, int KH, int KW, int stride_h, int stride_w,
              int pad_h, int pad_w, int flags, void* d_y, void* stream);

/* ---- int8 Conv2d (implicit GEMM) ------------------------------------------------- */
/* Padding modes of a convolution (Lucid's padding_mode, lucid/nn/functional/conv.py:24-29). */
enum { LQ_PAD_ZEROS = 0, LQ_PAD_REFLECT = 1, LQ_PAD_REPLICATE = 2, LQ_PAD_CIRCULAR = 3 };

/* Weight codes w[Cout, Cin_g, KH, KW] (Lucid's weight_int8 of a quantized Conv2d,
 * lucid/nn/quantized/conv.py:92-100) in the layout the conv kernel reads: one row per output
 * channel, w_p[co][(kh * KW + kw) * Cp + c] with Cp = Cin_g rounded up to 16 (zero codes),
 * each row KH * KW * Cp bytes rounded up to a multiple of 128 (zero tail), and the code sums
 * d_w_sums[Cout] (NULL to skip) for the activation zero-point term.  Built once per module.
 * No reference counterpart (a device layout; the state_dict keeps weight_int8). */
size_t lq_conv2d_weight_pack_size(int64_t Cout, int64_t Cin_g, int64_t KH, int64_t KW);
int lq_conv2d_pack_weights_i8(const int8_t* d_w, int64_t Cout, int64_t Cin_g, int64_t KH, int64_t KW,
                              int8_t* d_w_packed, int32_t* d_w_sums, void* stream);
/* Quantized Conv2d forward on activation codes x[N, C, H, W] (LQ_I8, or LQ_U8S8 for an
 * unsigned grid with d_a_zero_point its own zero point) and packed weights:
 *   acc[n, co, oh, ow] = sum_{c, kh, kw} (x[n, g*Cg + c, oh*sh + kh*dh - pt, ow*sw + kw*dw - pl] - za)
 *                        * w[co, c, kh, kw]                  (exact int32, padded taps = za)
 * then the epilogue of lq_gemm_w8a8 with a per-tensor activation scale, per-channel weight
 * scales d_w_scale[Cout] (symmetric weights: no weight zero point), bias, LQ_EPI_RELU and
 * out_kind, written NCHW to d_y[N, Cout, OH, OW].  Replaces dequantize -> F.conv2d ->
 * fake_quantize of lucid/nn/quantized/conv.py:137-172 (-> lucid/nn/functional/conv.py:53-84
 * -> lucid/_C/backend/cpu/methods/Conv.cpp:271-360).  padding_mode LQ_PAD_*; workspace of
 * lq_conv2d_i8_workspace_size bytes (same arguments as the call: the padded NHWC copy of x,
 * plus the int32 tile sums of a split K when the output has fewer tiles than the GPU has
 * CUs).  Two launches (three with a split K). */
size_t lq_conv2d_i8_workspace_size(int64_t N, int64_t C, int64_t H, int64_t W, int64_t Cout, int64_t KH, int64_t KW,
                                   int stride_h, int stride_w, int pad_top, int pad_bottom, int pad_left,
                                   int pad_right, int dilation_h, int dilation_w, int64_t groups);
int lq_conv2d_i8(const int8_t* d_x, int x_code_type, int64_t N, int64_t C, int64_t H, int64_t W,
                 const int8_t* d_w_packed, const int32_t* d_w_sums, int64_t Cout, int64_t KH, int64_t KW,
                 int stride_h, int stride_w, int pad_top, int pad_bottom, int pad_left, int pad_right,
                 int dilation_h, int dilation_w, int64_t groups, int padding_mode, const float* d_a_scale,
                 const float* d_a_zero_point, const float* d_w_scale, const float* d_bias,
                 const float* d_out_scale, const float* d_out_zero_point, int out_qmin, int out_qmax,
                 int out_kind, int flags, void* d_y, void* d_workspace, size_t workspace_bytes, void* stream);

/* The same convolution (groups 1, zeros padding, no dilation) between activations held in the
 * layout the implicit GEMM reads, for a network whose layers feed each other without
 * repacking: x is [N][H + 2 x_pad][W + 2 x_pad][x_cs] codes (x_cs = C rounded up to 16; the
 * border, x_pad >= pad, and the channel padding hold the activation zero point's code), and the
 * output is written the same way, y [N][OH + 2 y_pad][OW + 2 y_pad][y_cs] (y_pad 0 or 1; the
 * border filled with the output grid's zero-point code; Cout a multiple of 16), codes of
 * out_kind LQ_OUT_Q8 / QU8 / QU8S8.  With d_skip (codes of skip_type, the output's layout and
 * grid d_skip_scale / d_skip_zero_point) each output code c is then merged as lq_qmerge's
 * LQ_MERGE_ADD computes it -- fl32((c - z) s) + fl32((skip - zs) ss), ReLU with merge_flags
 * LQ_EPI_RELU, requantized to the merge grid (d_merge_scale / zero point, [merge_qmin,
 * merge_qmax], merge_type) -- the residual add of a quantized block (QFunctional.add_relu,
 * lucid/nn/quantized/functional_module.py:215-217) fused into its second convolution, and the
 * border holds the merge grid's zero point.  The bits of lq_conv2d_i8 followed by lq_qmerge on
 * the NCHW forms.  Workspace: lq_conv2d_i8_nhwc_workspace_size bytes (split-K sums; may be 0).
 * No reference counterpart: a device layout between Lucid's NCHW modules. */
size_t lq_conv2d_i8_nhwc_workspace_size(int64_t N, int64_t C, int64_t H, int64_t W, int64_t Cout, int64_t KH,
                                        int64_t KW, int stride, int pad);
int lq_conv2d_i8_nhwc(const int8_t* d_x, int x_code_type, int64_t N, int64_t C, int64_t H, int64_t W, int x_pad,
                      int64_t x_cs, const int8_t* d_w_packed, const int32_t* d_w_sums, int64_t Cout, int64_t KH,
                      int64_t KW, int stride, int pad, const float* d_a_scale, const float* d_a_zero_point,
                      const float* d_w_scale, const float* d_bias, const float* d_out_scale,
                      const float* d_out_zero_point, int out_qmin, int out_qmax, int out_kind, int flags, int8_t* d_y,
                      int y_pad, int64_t y_cs, const int8_t* d_skip, int skip_type, const float* d_skip_scale,
                      const float* d_skip_zero_point, const float* d_merge_scale, const float* d_merge_zero_point,
                      int merge_qmin, int merge_qmax, int merge_type, int merge_flags, void* d_workspace,
                      size_t workspace_bytes, void* stream);

/* Max pooling of byte codes (LQ_I8 / LQ_U8 / LQ_U8S8) from x[N, C, H, W] into the padded NHWC
 * layout of lq_conv2d_i8_nhwc: y [N][OH + 2 y_pad][OW + 2 y_pad][C] (y_cs == C, C a multiple
 * of 16, y_pad 0 or 1), the border filled with the code of *d_zero_point (the grid's zero
 * point; pooling keeps the grid).  Windows up to 3 x 3 with lq_pool2d's rules; the codes are
 * lq_pool2d's LQ_POOL_MAX.  Replaces max_pool2d over a quantized activation
 * (lucid/_C/backend/cpu/Pool.cpp:27-80) where the next layer reads the NHWC layout. */
int lq_maxpool2d_i8_to_nhwc(const int8_t* d_x, int x_type, const float* d_zero_point, int64_t N, int64_t C,
                            int64_t H, int64_t W, int64_t OH, int64_t OW, int KH, int KW, int stride_h, int stride_w,
                            int pad_h, int pad_w, int8_t* d_y, int y_pad, int64_t y_cs, void* stream);
/* Max pooling within that layout: x [N][H + 2 x_pad][W + 2 x_pad][x_cs] to y [N][OH + 2 y_pad]
 * [OW + 2 y_pad][y_cs] (C and both channel strides multiples of 16, windows up to 3 x 3, the
 * input border never read, the output border filled with the code of *d_zero_point); the codes
 * of lq_pool2d's LQ_POOL_MAX. */
int lq_maxpool2d_i8_nhwc(const int8_t* d_x, int x_type, const float* d_zero_point, int64_t N, int64_t C, int64_t H,
                         int64_t W, int x_pad, int64_t x_cs, int64_t OH, int64_t OW, int KH, int KW, int stride_h,
                         int stride_w, int pad_h, int pad_w, int8_t* d_y, int y_pad, int64_t y_cs, void* stream);
/* y[n, c] (float32 [N, C]) = the adaptive average pool to 1 x 1 of byte codes held in the padded
 * NHWC layout (x_pad border, x_cs bytes per pixel): sum over h, then w, of
 * fl32(fl32(float(c) - z) s), divided by H W -- lq_pool2d's LQ_POOL_AVG | LQ_POOL_ADAPTIVE bits
 * (lucid/nn/functional/_pool_core.py:407-434). */
int lq_avgpool2d_global_nhwc(const int8_t* d_x, int x_type, const float* d_scale, const float* d_zero_point,
                             int64_t N, int64_t C, int64_t H, int64_t W, int x_pad, int64_t x_cs, float* d_y,
                             void* stream);

/* ---- float helpers around the quantized path ----------------------------------- */
/* Float Conv2d y[N, Cout, OH, OW] (direct; the float model's conv during calibration,
 * lucid/nn/functional/conv.py:53-84 -> Conv.cpp:271-360): per output, sum over (c, kh, kw)
 * in that order in float32 (multiply then add), bias last. */
int lq_conv2d_f32(const float* d_x, int64_t N, int64_t C, int64_t H, int64_t W, const float* d_w,
                  const float* d_bias, int64_t Cout, int64_t KH, int64_t KW, int stride_h, int stride_w,
                  int pad_top, int pad_bottom, int pad_left, int pad_right, int dilation_h, int dilation_w,
                  int64_t groups, int padding_mode, float* d_y, void* stream);
/* Eval BatchNorm over [N, C, HW]: y = ((x - mean) * (1 / sqrt(var + eps))) * gamma + beta
 * (gamma / beta NULL: 1 / 0).  The float model's BatchNorm2d before fusion. */
int lq_batch_norm_f32(const float* d_x, float* d_y, int64_t N, int64_t C, int64_t HW, const float* d_mean,
                      const float* d_var, const float* d_gamma, const float* d_beta, float eps, void* stream);
/* y[i] = x[i] converted between LQ_F32, LQ_F16 and LQ_BF16 (round to nearest even when
 * narrowing; exact when widening), n elements; x and y may not overlap unless equal with
 * equal types.  Replaces astype_op (lucid/_C/ops/ufunc/Astype.cpp:42) between float types. */
int lq_cast(const void* d_x, int x_dtype, void* d_y, int y_dtype, int64_t n, void* stream);
/* y = (x <= 0) ? +0 : x, NaN passes (the CPU relu of backend/cpu/Vdsp.cpp vrelu_f32,
 * reached from nn.ReLU between quantized layers). */
int lq_relu_f32(const float* d_x, float* d_y, int64_t n, void* stream);
/* Float Linear y[M,N] = x[M,K] W[N,K]^T + bias (linear_op, lucid/_C/nn/Linear.cpp:199 ->
 * backend/cpu/methods/Matmul.cpp:80-122); runs the float model during calibration. */
int lq_linear_f32(const float* d_x, int64_t ldx, const float* d_w, int64_t ldw,
                  const float* d_bias, float* d_y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                  void* stream);

/* ---- float glue of a dynamically quantized transformer ---- */
/* Kernels a decoder runs between its int8 Linears, each a float32 restatement of a Lucid
 * float module; compared with float64 within tolerance.
 * Positions: where an entry point takes (pos0, d_pos0), the first token's position is pos0,
 * or d_pos0[0] when d_pos0 is not NULL (a device counter, so one captured decode step replays
 * at every position; kernels clamp it into range, the caller keeps it valid). */
/* out[r] = tok_table[clamp(tokens[r])] + pos_table[pos + r % n] for rows = B * n token rows
 * (nn.Embedding lookups plus the positional add); pos_table has npos rows. */
int lq_embedding_sum_f32(const float* d_tok_table, int64_t vocab, const float* d_pos_table, int64_t npos, int64_t D,
                         const int32_t* d_tokens, int64_t rows, int64_t n, int64_t pos0, const int32_t* d_pos0,
                         float* d_out, void* stream);
/* y = (x - mean) / sqrt(var + eps) (* gamma + beta when given) per row of D (nn.LayerNorm,
 * biased variance); rows ldx / ldy elements apart. */
int lq_layer_norm_f32(const float* d_x, int64_t ldx, float* d_y, int64_t ldy, int64_t rows, int64_t D,
                      const float* d_gamma, const float* d_beta, float eps, void* stream);
/* x = x + res, then y = lq_layer_norm_f32(x) per row (a pre-norm block's residual add fused with
 * the next norm: the same bits as lq_add_f32 followed by lq_layer_norm_f32, one launch); rows
 * ldx / ldres / ldy elements apart, y must not overlap x or res. */
int lq_add_layer_norm_f32(float* d_x, int64_t ldx, const float* d_res, int64_t ldres, float* d_y, int64_t ldy,
                          int64_t rows, int64_t D, const float* d_gamma, const float* d_beta, float eps,
                          void* stream);
/* y = 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) (F.gelu, approximate="tanh"), evaluated as
 * x / (1 + exp(-2 sqrt(2/pi) (x + 0.044715 x^3))) with the hardware exp2 and reciprocal (the same
 * function, within a few float32 ulps). */
int lq_gelu_tanh_f32(const float* d_x, float* d_y, int64_t n, void* stream);
/* y = a + b elementwise (residual adds). */
int lq_add_f32(const float* d_a, const float* d_b, float* d_y, int64_t n, void* stream);
/* y = a + fl32(b * s), each operation rounded once: a LoRA layer's output plus its scaled
 * low-rank update, and a merge's weight plus the scaled delta
 * (lucid/peft/tuners/lora/_layer.py:796-803, 971-989). */
int lq_add_scaled_f32(const float* d_a, const float* d_b, float s, float* d_y, int64_t n, void* stream);
/* y [cols, rows] = x [rows, cols]^T (float32; y must not alias x). */
int lq_transpose_f32(const float* d_x, int64_t rows, int64_t cols, float* d_y, void* stream);
/* qkv [B, n, 3, H, hd] float32 -> q [B, H, n, hd] fp16, and k / v written into the fp16
 * caches [B, H, T_max, hd] at positions pos .. pos + n - 1. */
int lq_kv_append_f16(const float* d_qkv, int64_t B, int64_t n, int64_t H, int64_t hd, int64_t pos0,
                     const int32_t* d_pos0, int64_t T_max, void* d_q, void* d_k_cache, void* d_v_cache, void* stream);
/* The same layout change from an fp16 qkv (the projection's LQ_OUT_F16 output: each value the
 * fp16 rounding of the float32 one, so the caches and q hold the bits lq_kv_append_f16 writes
 * from the float32 output) -- half the bytes read, no conversion.  hd % 8 == 0, 16-byte aligned
 * buffers. */
int lq_kv_append_h16(const void* d_qkv, int64_t B, int64_t n, int64_t H, int64_t hd, int64_t pos0,
                     const int32_t* d_pos0, int64_t T_max, void* d_q, void* d_k_cache, void* d_v_cache, void* stream);
/* Causal attention over the fp16 cache (F.scaled_dot_product_attention, is_causal): query i of
 * q [B, H, n, hd] sits at position pos + i and sees keys 0 .. pos + i; softmax(scale q.k) v
 * with fp32 scores and sums (fp16 MFMA products for n > 1); out [B, n, H, hd] float32.
 * hd = 64; a single query (n = 1) sees at most 2048 keys (LQ_ERR_UNSUPPORTED otherwise). */
int lq_attention_f16(const void* d_q, const void* d_k_cache, const void* d_v_cache, int64_t B, int64_t H, int64_t n,
                     int64_t hd, int64_t pos0, const int32_t* d_pos0, int64_t T_max, float scale, float* d_out,
                     void* stream);
/* lq_attention_f16, then lq_dynamic_quantize_f32 of its output [B, n, H, hd] into codes and
 * d_qparams {min, max, scale, zero point}: the input step of the dynamic out-projection after
 * attention (lucid/nn/quantized/dynamic/linear.py:85-92), the same bits as the two calls.  For
 * n > 1 (the flash kernel) above 16384 values with aligned output and codes, the attention folds
 * the extrema of what it stores per workgroup and the quantize folds those pairs: two launches
 * where the calls take three.  Workspace: lq_attention_dynamic_quantize_workspace_size bytes. */
size_t lq_attention_dynamic_quantize_workspace_size(int64_t B, int64_t H, int64_t n, int64_t hd);
int lq_attention_dynamic_quantize_f16(const void* d_q, const void* d_k_cache, const void* d_v_cache, int64_t B,
                                      int64_t H, int64_t n, int64_t hd, int64_t pos0, const int32_t* d_pos0,
                                      int64_t T_max, float scale, float* d_out, int q_dtype, int qmin, int qmax,
                                      float eps, float* d_qparams, void* d_codes, void* d_workspace,
                                      size_t workspace_bytes, void* stream);
/* One decode step's lq_kv_append_f16 + lq_attention_f16 (n = 1) in one launch: qkv [B, 1, 3,
 * H, hd] float32; k / v rounded to fp16 into the caches at the position, q rounded to fp16,
 * then the attention of that query over keys 0 .. pos; out [B, 1, H, hd] float32.  Same
 * rounding of q / k / v as the two calls.  hd = 64, at most 2048 keys. */
int lq_kv_append_attention_f16(const float* d_qkv, int64_t B, int64_t H, int64_t hd, int64_t pos0,
                               const int32_t* d_pos0, int64_t T_max, void* d_k_cache, void* d_v_cache, float scale,
                               float* d_out, void* stream);
/* x[0] += delta (advances a device position counter inside a captured step). */
int lq_increment_i32(int32_t* d_x, int32_t delta, void* stream);
/* idx[r] = index of the first maximum of row r (numpy argmax; a NaN counts as the maximum). */
int lq_argmax_f32(const float* d_x, int64_t rows, int64_t cols, int32_t* d_idx, void* stream);
/* lq_argmax_f32 and lq_increment_i32(d_pos, delta) in one launch (the end of a decode step:
 * the greedy token and the position advance; the argmax does not read *d_pos). */
int lq_argmax_next_f32(const float* d_x, int64_t rows, int64_t cols, int32_t* d_idx, int32_t* d_pos, int32_t delta,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LQ_API_H */
