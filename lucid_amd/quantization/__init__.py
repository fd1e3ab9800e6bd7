"""``lucid_amd.quantization``: Lucid's quantization API (lucid/quantization/__init__.py:36-126)
on the HIP backend."""

from lucid_amd.quantization._functional import dequantize, fake_quantize, quantize
from lucid_amd.quantization._qparams import QParams, calculate_qparams
from lucid_amd.quantization._qscheme import (
    QDtype,
    QScheme,
    per_channel_affine,
    per_channel_symmetric,
    per_tensor_affine,
    per_tensor_symmetric,
    qint4,
    qint8,
    qint32,
    quint8,
)
from lucid_amd.quantization.observer import (
    FixedQParamsObserver,
    HistogramObserver,
    MinMaxObserver,
    MovingAverageMinMaxObserver,
    MovingAveragePerChannelMinMaxObserver,
    NoopObserver,
    ObserverBase,
    PerChannelMinMaxObserver,
    PlaceholderObserver,
)
from lucid_amd.quantization.qconfig import (
    QConfig,
    QConfigMapping,
    get_default_qconfig,
    get_default_qconfig_mapping,
    get_minmax_qconfig,
)
from lucid_amd.quantization._quantize import convert, prepare, quantize_dynamic
from lucid_amd.quantization.fuse_modules import fuse_modules

__all__ = [
    "QScheme", "per_tensor_affine", "per_tensor_symmetric", "per_channel_affine",
    "per_channel_symmetric", "QDtype", "qint8", "quint8", "qint32", "qint4", "QParams",
    "calculate_qparams", "quantize", "dequantize", "fake_quantize", "ObserverBase",
    "MinMaxObserver", "MovingAverageMinMaxObserver", "PerChannelMinMaxObserver",
    "MovingAveragePerChannelMinMaxObserver", "HistogramObserver", "FixedQParamsObserver",
    "PlaceholderObserver", "NoopObserver", "QConfig", "QConfigMapping", "get_default_qconfig",
    "get_default_qconfig_mapping", "get_minmax_qconfig", "prepare", "convert", "quantize_dynamic",
    "fuse_modules",
]
