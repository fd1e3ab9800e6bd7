"""lucid_amd -- Lucid's int8 quantized-inference path as an MI355X (gfx950) HIP backend.

The Python surface mirrors ``lucid.quantization``, ``lucid.nn.quantized`` and
``lucid.backends.quantized`` (names, arguments, ``state_dict`` layouts); every op runs as a
hand-written HIP kernel behind the C ABI of ``include/lq_api.h``.  There is no CPU
fallback: device ops on CPU tensors raise, and a missing backend library raises
:class:`BackendUnavailable` on first use.
"""

from lucid_amd import _C
from lucid_amd._C import BackendUnavailable, LucidError, is_available, synchronize
from lucid_amd._tensor import (
    QuantSource,
    Tensor,
    bf16_from_f32,
    bf16_to_f32,
    bfloat16,
    bool_,
    dtype,
    empty,
    float16,
    float32,
    float64,
    from_numpy,
    full,
    int8,
    int16,
    int32,
    int64,
    ones,
    randn,
    tensor,
    uint8,
    uint32,
    zeros,
    zeros_like,
)

__version__ = "0.1.0"


def __getattr__(name: str):
    # Sub-packages load lazily so `import lucid_amd` stays cheap and import cycles stay out.
    import importlib

    if name in ("nn", "quantization", "backends", "serialization"):
        return importlib.import_module(f"lucid_amd.{name}")
    if name in ("save", "load"):  # lucid.save / lucid.load
        return getattr(importlib.import_module("lucid_amd.serialization"), name)
    raise AttributeError(f"module 'lucid_amd' has no attribute {name!r}")
