"""ctypes binding of the HIP backend library (``include/lq_api.h``).

This is the thin shim between Lucid's Python op/module surface and the gfx950
kernels, in the place of Lucid's pybind seam ``_C_engine.quantized``
(lucid/_C/bindings/bind_quantized.cpp:17-27).  Loading fails loudly: there is
no CPU fallback, so a missing or unloadable ``liblucid_amd.so`` raises
:class:`BackendUnavailable` and a device call without a GPU raises
:class:`LucidError`.
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "liblucid_amd.so")

# Status and type codes of include/lq_api.h.
OK = 0
I8, U8, I16, I32, F16, F32, U8S8, I64 = 1, 2, 3, 4, 5, 6, 7, 8
I8_QPAIR = 9  # table lookups: int8 rows + interleaved {scale, zero point} pairs
BF16 = 10
OBS_MINMAX, OBS_EMA, OBS_REPLACE = 0, 1, 2
OUT_I32, OUT_F32, OUT_F16, OUT_Q8, OUT_QU8, OUT_FQ32, OUT_Q16, OUT_QU8S8 = 0, 1, 2, 3, 4, 5, 6, 7
EPI_RELU, EPI_A_U8S8, EPI_ROUND_BF16, EPI_GELU = 1, 2, 4, 8
CONV_OUT_NHWC = 16
DL_PLAIN, DL_LN, DL_ADD_LN = 0, 1, 2
PAD_ZEROS, PAD_REFLECT, PAD_REPLICATE, PAD_CIRCULAR = 0, 1, 2, 3
MERGE_ADD, MERGE_MUL, MERGE_ADD_SCALAR, MERGE_MUL_SCALAR, MERGE_COPY = 0, 1, 2, 3, 4
ACT_SIGMOID, ACT_TANH, ACT_HARDSWISH, ACT_HARDSIGMOID, ACT_ELU, ACT_LEAKY_RELU = 0, 1, 2, 3, 4, 5
BAG_SUM, BAG_MEAN, BAG_MAX = 0, 1, 2
POOL_MAX, POOL_AVG = 0, 1
RNN_TANH, RNN_RELU, RNN_LSTM, RNN_GRU = 0, 1, 2, 3
POOL_ADAPTIVE, POOL_COUNT_INCLUDE_PAD = 1, 2


class LucidError(RuntimeError):
    """Error raised by the backend (the role of Lucid's ``LucidError``, bind_errors.cpp:6-71)."""


class BackendUnavailable(LucidError):
    """The HIP backend library is missing or cannot be loaded."""


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float
_I = ctypes.c_int
_SZ = ctypes.c_size_t

# name -> (restype, argtypes)
_SIGNATURES: dict[str, tuple] = {
    "lq_abi_version": (_I, []),
    "lq_last_error": (ctypes.c_char_p, []),
    "lq_last_path": (ctypes.c_char_p, []),
    "lq_backend_name": (ctypes.c_char_p, []),
    "lq_device_count": (_I, [ctypes.POINTER(_I)]),
    "lq_set_device": (_I, [_I]),
    "lq_get_device": (_I, [ctypes.POINTER(_I)]),
    "lq_malloc": (_I, [ctypes.POINTER(_P), _SZ]),
    "lq_free": (_I, [_P]),
    "lq_malloc_async": (_I, [ctypes.POINTER(_P), _SZ, _P]),
    "lq_free_async": (_I, [_P, _P]),
    "lq_record_stream": (_I, [_P, _P]),
    "lq_empty_cache": (_I, []),
    "lq_memory_stats": (_I, [ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]),
    "lq_memcpy_h2d": (_I, [_P, _P, _SZ, _P]),
    "lq_memcpy_d2h": (_I, [_P, _P, _SZ, _P]),
    "lq_memcpy_d2d": (_I, [_P, _P, _SZ, _P]),
    "lq_fill_u32": (_I, [_P, ctypes.c_uint32, _SZ, _P]),
    "lq_read_floor": (_I, [_P, _SZ, ctypes.c_uint32, _P, _P]),
    "lq_stream_create": (_I, [ctypes.POINTER(_P)]),
    "lq_stream_destroy": (_I, [_P]),
    "lq_stream_synchronize": (_I, [_P]),
    "lq_device_synchronize": (_I, []),
    "lq_event_create": (_I, [ctypes.POINTER(_P)]),
    "lq_event_destroy": (_I, [_P]),
    "lq_event_record": (_I, [_P, _P]),
    "lq_event_synchronize": (_I, [_P]),
    "lq_event_elapsed_ms": (_I, [ctypes.POINTER(_F), _P, _P]),
    "lq_histc_workspace_size": (_SZ, [_I64]),
    "lq_histc_f32": (_I, [_P, _I64, _I64, ctypes.c_double, ctypes.c_double, _I, _P, _P, _SZ, _P]),
    "lq_hist_rebin_f32": (_I, [_P, _I64, _F, _F, _F, _F, _P, _P]),
    "lq_embedding": (_I, [_P, _I, _P, _P, _I64, _I64, _P, _I, _I64, _P, _P]),
    "lq_embedding_bag": (_I, [_P, _I, _P, _P, _I64, _I64, _P, _I, _I64, _P, _I, _I64, _I, _I64, _I, _I64, _P, _P,
                              _P]),
    "lq_pool2d": (_I, [_I, _P, _I, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I, _I, _I, _I, _I, _I, _P, _P]),
    "lq_rnn_cell": (_I, [_I, _P, _I64, _P, _I64, _P, _P, _I64, _I64, _P, _P, _P, _I64, _P]),
    "lq_stride_expand": (_I, [_P, _I, _I64, _I64, _I64, _I, _I, _P, _P, _P]),
    "lq_depth_gather": (_I, [_P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P,
                             _P, _P]),
    "lq_permute_0213": (_I, [_P, _I, _I64, _I64, _I64, _I64, _P, _P]),
    "lq_qact": (_I, [_I, _P, _I, _P, _P, _I64, _F, _P, _P, _I, _I, _I, _P, _P]),
    "lq_qmerge": (_I, [_I, _P, _I, _P, _P, _P, _I, _P, _P, _F, _I64, _I64, _I64, _P, _P, _I, _I, _I, _I,
                       _P, _P]),
    "lq_graph_begin_capture": (_I, [_P]),
    "lq_graph_end_capture": (_I, [_P, ctypes.POINTER(_P)]),
    "lq_graph_launch": (_I, [_P, _P]),
    "lq_graph_destroy": (_I, [_P]),
    "lq_minmax_workspace_size": (_SZ, [_I64]),
    "lq_minmax_f32": (_I, [_P, _I64, _P, _P, _I, _F, _P, _SZ, _P]),
    "lq_minmax_per_channel_workspace_size": (_SZ, [_I64, _I64, _I64]),
    "lq_minmax_per_channel_f32": (_I, [_P, _I64, _I64, _I64, _P, _P, _I, _F, _P, _SZ, _P]),
    "lq_calc_qparams_f32": (_I, [_P, _P, _I64, _I, _I, _I, _I, _F, _P, _P, _P]),
    "lq_quantize_per_tensor_f32": (_I, [_P, _P, _I64, _I, _P, _P, _F, _F, _I, _I, _P]),
    "lq_dynamic_quantize_workspace_size": (_SZ, [_I64]),
    "lq_dynamic_quantize_f32": (_I, [_P, _I64, _I, _I, _I, _F, _P, _P, _P, _SZ, _P]),
    "lq_layer_norm_quantize_f32": (_I, [_P, _I64, _P, _I64, _I64, _I64, _P, _P, _F, _I, _I, _I, _F, _P, _P, _P]),
    "lq_layer_norm_dynamic_quantize_workspace_size": (_SZ, [_I64, _I64]),
    "lq_layer_norm_dynamic_quantize_f32": (_I, [_P, _I64, _P, _I64, _I64, _I64, _P, _P, _F, _P, _I, _I, _I, _F, _P, _P,
                                               _P, _SZ, _P]),
    "lq_quantize_per_channel_f32": (_I, [_P, _P, _I64, _I64, _I64, _I, _P, _P, _F, _I, _I, _P]),
    "lq_dequantize_per_tensor": (_I, [_P, _I, _P, _I, _I64, _P, _P, _F, _F, _P]),
    "lq_dequantize_per_channel": (_I, [_P, _I, _P, _I, _I64, _I64, _I64, _P, _P, _F, _P]),
    "lq_fake_quantize_per_tensor_f32": (_I, [_P, _P, _I64, _P, _P, _F, _F, _F, _I, _I, _P, _P]),
    "lq_fake_quantize_per_channel_f32": (_I, [_P, _P, _I64, _I64, _I64, _P, _P, _F, _I, _I, _P, _P]),
    "lq_row_sums_i8": (_I, [_P, _I64, _I64, _I64, _P, _P]),
    "lq_gemm_w8a8_workspace_size": (_SZ, [_I64, _I64, _I64]),
    "lq_gemm_w8a8": (_I, [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P, _I64,
                          _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _SZ, _P]),
    "lq_gemm_w8a8_noalloc_scratch_bytes": (_SZ, []),
    "lq_gemm_w8a8_noalloc": (_I, [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P, _I64,
                                  _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "lq_embedding_sum_f32": (_I, [_P, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64, _P, _P, _P]),
    "lq_layer_norm_f32": (_I, [_P, _I64, _P, _I64, _I64, _I64, _P, _P, _F, _P]),
    "lq_add_layer_norm_f32": (_I, [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P, _P, _F, _P]),
    "lq_gelu_tanh_f32": (_I, [_P, _P, _I64, _P]),
    "lq_add_f32": (_I, [_P, _P, _P, _I64, _P]),
    "lq_add_scaled_f32": (_I, [_P, _P, _F, _P, _I64, _P]),
    "lq_transpose_f32": (_I, [_P, _I64, _I64, _P, _P]),
    "lq_kv_append_f16": (_I, [_P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _P]),
    "lq_kv_append_h16": (_I, [_P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _P]),
    "lq_attention_dynamic_quantize_workspace_size": (_SZ, [_I64, _I64, _I64, _I64]),
    "lq_gemm_w8a8_dynamic_quantize_workspace_size": (_SZ, [_I64, _I64, _I64]),
    "lq_gemm_w8a8_dynamic_quantize": (_I, [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _P, _P,
                                           _P, _I, _I, _I, _I, _F, _P, _P, _P, _SZ, _P]),
    "lq_attention_dynamic_quantize_f16": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _F, _P, _I, _I,
                                               _I, _F, _P, _P, _P, _SZ, _P]),
    "lq_attention_f16": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _F, _P, _P]),
    "lq_increment_i32": (_I, [_P, ctypes.c_int32, _P]),
    "lq_argmax_f32": (_I, [_P, _I64, _I64, _P, _P]),
    "lq_argmax_next_f32": (_I, [_P, _I64, _I64, _P, _P, ctypes.c_int32, _P]),
    "lq_kv_append_attention_f16": (_I, [_P, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _F, _P, _P]),
    "lq_packed_weights_size": (_SZ, [_I64, _I64]),
    "lq_pack_weights_i8": (_I, [_P, _I64, _I64, _I64, _P, _P]),
    "lq_gemm_w8a8_packed": (_I, [_P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _P, _I64,
                                 _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _SZ, _P]),
    "lq_dynamic_linear_packed_f32": (_I, [_P, _I64, _P, _I64, _P, _I64, _I, _P, _P, _F, _I64, _I64, _I, _I, _F,
                                          _P, _P, _P, _P, _P, _I64, _P, _I64, _I, _P]),
    "lq_conv2d_i8_nhwc_workspace_size": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I]),
    "lq_conv2d_i8_nhwc": (_I, [_P, _I, _I64, _I64, _I64, _I64, _I, _I64, _P, _P, _I64, _I64, _I64, _I, _I, _P, _P,
                               _P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _I64, _P, _I, _P, _P, _P, _P, _I, _I, _I,
                               _I, _P, _SZ, _P]),
    "lq_maxpool2d_i8_to_nhwc": (_I, [_P, _I, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I, _I, _I, _I, _I, _P, _I,
                                     _I64, _P]),
    "lq_avgpool2d_global_nhwc": (_I, [_P, _I, _P, _P, _I64, _I64, _I64, _I64, _I, _I64, _P, _P]),
    "lq_maxpool2d_i8_nhwc": (_I, [_P, _I, _P, _I64, _I64, _I64, _I64, _I, _I64, _I64, _I64, _I, _I, _I, _I, _I, _I,
                                  _P, _I, _I64, _P]),
    "lq_conv2d_weight_pack_size": (_SZ, [_I64, _I64, _I64, _I64]),
    "lq_conv2d_pack_weights_i8": (_I, [_P, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "lq_conv2d_i8_workspace_size": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I, _I, _I, _I, _I, _I, _I,
                                          _I64]),
    "lq_conv2d_i8": (_I, [_P, _I, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64, _I, _I, _I, _I, _I,
                          _I, _I, _I, _I64, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _SZ,
                          _P]),
    "lq_conv2d_f32": (_I, [_P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64, _I, _I, _I, _I, _I, _I,
                           _I, _I, _I64, _I, _P, _P]),
    "lq_batch_norm_f32": (_I, [_P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _F, _P]),
    "lq_cast": (_I, [_P, _I, _P, _I, _I64, _P]),
    "lq_gemv_w8_workspace_size": (_SZ, [_I64, _I64, _I64]),
    "lq_gemv_w8": (_I, [_P, _I, _I64, _P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _P,
                        _SZ, _P]),
    "lq_gemv_w8_packed_workspace_size": (_SZ, [_I64, _I64, _I64]),
    "lq_gemv_w8_packed": (_I, [_P, _I, _I64, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _SZ, _P]),
    "lq_group_quantize_f32": (_I, [_P, _I64, _I64, _I, _I, _P, _P, _P, _P]),
    "lq_group_dequantize_f32": (_I, [_P, _P, _P, _I64, _I64, _I, _I, _P, _P]),
    "lq_group_matmul_workspace_size": (_SZ, [_I64, _I64, _I64, _I]),
    "lq_group_matmul": (_I, [_P, _I, _I64, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _I,
                             _I, _I, _P, _SZ, _P]),
}

_lib = None
_lib_lock = threading.Lock()


def _declare(L: ctypes.CDLL, sigs: dict[str, tuple]) -> None:
    for name, (res, args) in sigs.items():
        fn = getattr(L, name, None)
        if fn is None:
            raise BackendUnavailable(f"{LIB_PATH} does not export {name}")
        fn.restype = res
        fn.argtypes = args


def register_signatures(sigs: dict[str, tuple]) -> None:
    """Add entry points declared by another module (kept beside their wrappers)."""
    _SIGNATURES.update(sigs)
    if _lib is not None:
        _declare(_lib, sigs)


def lib() -> ctypes.CDLL:
    """The loaded backend library; raises :class:`BackendUnavailable` if absent."""
    global _lib
    if _lib is None:
        with _lib_lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise BackendUnavailable(
                        f"HIP backend library not built: {LIB_PATH} is missing "
                        "(run `python -m lucid_amd.build`)"
                    )
                try:
                    L = ctypes.CDLL(LIB_PATH)
                except OSError as e:
                    raise BackendUnavailable(f"cannot load {LIB_PATH}: {e}") from e
                _declare(L, _SIGNATURES)
                if L.lq_abi_version() != 1:
                    raise BackendUnavailable("ABI version mismatch")
                _lib = L
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc != OK:
        msg = lib().lq_last_error().decode(errors="replace")
        raise LucidError(f"{what}: {msg}" if what else msg)


_entry_points: dict = {}


_recording: list | None = None  # (name, args) of every call while a capture records (lucid_amd.graphs)


def call(name: str, *args) -> None:
    """Call an int-status entry point and raise on failure (the ctypes function object is
    looked up once per name)."""
    f = _entry_points.get(name)
    if f is None:
        f = _entry_points[name] = getattr(lib(), name)
    if _recording is not None:
        _recording.append((name, args))
    rc = f(*args)
    if rc != OK:
        check(rc, name)


def last_path() -> str:
    """Kernel variant the last GEMM / convolution call on this thread launched."""
    return lib().lq_last_path().decode()


def device_count() -> int:
    n = _I(0)
    check(lib().lq_device_count(ctypes.byref(n)), "lq_device_count")
    return n.value


def is_available() -> bool:
    """True when the library loads and a GPU is visible."""
    try:
        return device_count() > 0
    except LucidError:
        return False


def synchronize() -> None:
    check(lib().lq_device_synchronize(), "lq_device_synchronize")
