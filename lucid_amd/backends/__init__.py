"""``lucid_amd.backends.quantized``: the quantized engine selector
(lucid/backends/__init__.py:57-113).

``engine`` is ``"auto"``, ``"mlx_group"`` or ``"reference"``, the values Lucid accepts.
``use_mlx()`` decides whether ``convert`` / ``quantize_dynamic`` route the Linear family to
the group-wise weight-only layer: ``"reference"`` never does, ``"mlx_group"`` always does,
``"auto"`` does when that layer is ``available`` on this backend.  ``available`` is true
when the HIP library loads, a GPU is present and the group-wise kernels are exported.
"""

from __future__ import annotations

from typing import final as _final

_GROUP_SYMBOLS = ("lq_group_quantize_f32", "lq_group_dequantize_f32", "lq_group_matmul")


@_final
class _QuantizedBackend:
    _engine: str = "auto"

    @property
    def available(self) -> bool:
        from lucid_amd import _C

        try:
            lib = _C.lib()
        except Exception:
            return False
        if not all(hasattr(lib, s) for s in _GROUP_SYMBOLS):
            return False
        return _C.is_available()

    @property
    def engine(self) -> str:
        return self._engine

    @engine.setter
    def engine(self, value: str) -> None:
        if value not in ("auto", "mlx_group", "reference"):
            raise ValueError(
                f"quantized.engine must be 'auto'/'mlx_group'/'reference', got {value!r}")
        self._engine = value

    def use_mlx(self) -> bool:
        if self._engine == "reference":
            return False
        if self._engine == "mlx_group":
            return True
        return self.available


quantized = _QuantizedBackend()

__all__ = ["quantized"]
